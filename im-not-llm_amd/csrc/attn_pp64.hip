// Ping-pong bf16 attention for head_dim 64 (one K/V head per query head) on
// gfx950.
//
// The schedule of attn_pp.hip (persistent unit stream, two groups of 4 waves
// alternating barrier-separated MFMA and softmax phases on every SIMD, K/V
// tiles staged with direct loads, V converted to fp16 in place), with one
// difference: without grouped queries no two query heads share K and V, so
// each group streams the tiles of its own head. A work unit is one block of
// 128 query rows of one text for a pair of heads (2 hp, 2 hp + 1); group g
// serves head 2 hp + g with its own 4 LDS stages. Both heads have the same
// rows and masks, so both groups step through the same tiles in lockstep.
//
// LDS layout, per group (64 KB): 4 K stages then 4 V stages of 64 keys x
// 128 bytes.
//   K: 16-byte chunk c of key row r at r * 128 + ((c ^ ((r >> 1) & 7)) * 16);
//      a QK^T fragment read (16 rows at one logical chunk per 16 lanes)
//      touches all 16 chunk positions of a 256-byte bank row.
//   V: fp16, chunk c of row r at r * 128 + ((c ^ (((r >> 1) & 1) << 2)) * 16);
//      a transposed PV fragment read (8 rows x 64 bytes) puts two rows on
//      each 64-byte column group.
// Both swizzles are applied by choosing which global chunk each lane loads.

#include <type_traits>

#include "attn_stream.hpp"

namespace inl {

namespace {

template <int BN>
struct PP64Shape {
  static_assert(PP_MAX_UNITS % 4 == 0, "descriptor table alignment");
  static constexpr int D = 64;
  static constexpr int NT = 512;            // 8 waves, 2 groups of 4
  static constexpr int CH = D / 8;          // 16-byte chunks per row
  static constexpr int ROW = D * 2;         // bytes per K or V row in LDS
  static constexpr int TILE = BN * ROW;     // bytes per K (or V) stage
  static constexpr int STAGES = 4;
  static constexpr int VOFF = STAGES * TILE;     // V stages within a group
  static constexpr int GROUP = 2 * STAGES * TILE;
  static constexpr int TILES_LDS = 2 * GROUP;
  static constexpr int LDS = TILES_LDS + PP_MAX_UNITS * (16 + 4);
  static constexpr int KPW = TILE / 1024 / 4;  // 1 KB direct loads per wave per tile (K and V each)
  static constexpr int RPB = 1024 / ROW;       // rows per 1 KB block
  static_assert(KPW >= 1, "tile too small for 4 waves");
  static_assert(TILE == 8192, "output staging assumes 8 KB stages");
};

template <int BN>
__global__ __launch_bounds__(512, 1) void attn_pp64_kernel(AttnParams p) {
  using S = PP64Shape<BN>;
  constexpr int D = S::D;
  constexpr int NKB = BN / 32;   // 32-key blocks of S^T
  constexpr int NDB = D / 32;    // 32-wide d blocks of O^T
  constexpr int KST = D / 16;    // k-steps of the QK^T product
  constexpr int PKS = BN / 16;   // k-steps of the PV product

  extern __shared__ __attribute__((aligned(16))) char smem[];
  const uint32_t lds0 = lds_addr(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int wg = wave & 3;       // wave within its group
  const int lq = lane & 31;
  const int hf = lane >> 5;
  const uint32_t gl = lds0 + grp * S::GROUP;   // this group's stages

  // ---- this workgroup's work units (host-ordered), staged in LDS ----
  const int u_first = p.wg_start[blockIdx.x];
  const int nu = p.wg_start[blockIdx.x + 1] - u_first;
  if (nu <= 0) return;
  int4* const sdesc = reinterpret_cast<int4*>(smem + S::TILES_LDS);
  int* const shg = reinterpret_cast<int*>(sdesc + PP_MAX_UNITS);
  for (int i = tid; i < nu; i += S::NT) {
    sdesc[i] = p.items[u_first + i];
    shg[i] = p.unit_hg[u_first + i];
  }
  // The stream's first PV product reads V stage 3 with P = 0: zero it (both
  // groups), so that no stale LDS bits (NaN as fp16) reach the accumulator.
  for (int i = tid; i < 2 * S::TILE / 16; i += S::NT) {
    const int g = i / (S::TILE / 16), o = i % (S::TILE / 16);
    reinterpret_cast<u32x4*>(smem + g * S::GROUP + S::VOFF + (S::STAGES - 1) * S::TILE)[o] =
        (u32x4){0u, 0u, 0u, 0u};
  }
  __syncthreads();

  const int causal = p.causal;
  const int window = p.window;
  const uint32_t kst_b = (uint32_t)(p.k_stride * 2);
  const uint32_t vst_b = (uint32_t)(p.v_stride * 2);
  const uint32_t qst_b = (uint32_t)(p.q_stride * 2);
  const int osz = p.out_bf16 ? 2 : 4;

  // Unit u: {text start row, text length, first query row, lo_tile << 16 | hi_tile}
  // and its head pair; read wave-uniformly from LDS.
  auto unit = [&](int u, int& seg, int& T, int& q0, int& lo, int& hi, int& hp) __attribute__((always_inline)) {
    const int4 d = sdesc[u];
    seg = __builtin_amdgcn_readfirstlane(d.x);
    T = __builtin_amdgcn_readfirstlane(d.y);
    q0 = __builtin_amdgcn_readfirstlane(d.z);
    lo = (int)((uint32_t)__builtin_amdgcn_readfirstlane(d.w) >> 16);
    hi = __builtin_amdgcn_readfirstlane(d.w) & 0xffff;
    hp = __builtin_amdgcn_readfirstlane(shg[u]);
  };

  // ---- per-lane constant offsets ----
  // This wave's slice of its group's tiles: 1 KB blocks i * 4 + wg. Lane l of
  // a block fills LDS slot l: row blk * RPB + l / CH, physical chunk l % CH,
  // and so loads the logical chunk the swizzle puts there.
  uint32_t kg_off[S::KPW], vg_off[S::KPW];   // global byte offsets within a tile
  uint32_t cv_a[S::KPW];                      // LDS address of the stage-0 V chunk this lane converts
#pragma unroll
  for (int i = 0; i < S::KPW; ++i) {
    const int blk = i * 4 + wg;
    const int row = blk * S::RPB + lane / S::CH;
    const int pc = lane % S::CH;
    kg_off[i] = (uint32_t)row * kst_b + ((pc ^ ((row >> 1) & 7)) << 4);
    vg_off[i] = (uint32_t)row * vst_b + ((pc ^ (((row >> 1) & 1) << 2)) << 4);
    cv_a[i] = opaque(gl + S::VOFF + blk * 1024 + lane * 16);
  }
  // QK^T fragment of step st (rows lq, lq + 32): logical chunk 2 st + hf.
  uint32_t ka[KST];   // LDS address of the fragment in stage 0
#pragma unroll
  for (int st = 0; st < KST; ++st) ka[st] = opaque(gl + lq * S::ROW + (((2 * st + hf) ^ ((lq >> 1) & 7)) << 4));
  // PV fragment (db, ks, half): rows ks*16 + 8*half + vrow, logical columns
  // db*32 + vcol .. +3. The swizzle of those rows depends on bit 1 of vrow
  // only, so each db has one per-lane base and ks / half are immediate
  // offsets.
  const int g16 = lane >> 4;
  const int j16 = lane & 15;
  const int vcol = 16 * (g16 & 1) + 4 * (j16 & 3);
  const int vrow = 4 * hf + (j16 >> 2);
  uint32_t va[NDB];   // LDS address of the fragment in stage 0
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    va[db] = opaque(gl + S::VOFF + vrow * S::ROW +
                    ((((4 * db + (vcol >> 3)) ^ (((vrow >> 1) & 1) << 2)) << 4) | ((vcol * 2) & 15)));

  // ---- load cursor: the next tile of this group's tile stream to load ----
  // Every wave loads its slice of every tile of its head, in stream order,
  // into stage (stream index) % 4. Past the stream's end the descriptors get
  // an empty range: the loads still go out and return zeros into a stage
  // that no later phase reads.
  int du = 0, dt = 0, dhi = 0;
  i32x4 krs, vrs;
  auto dma_unit = [&](int u) __attribute__((always_inline)) {
    if (u < nu) {
      int seg, T, q0, lo, hi, hp;
      unit(u, seg, T, q0, lo, hi, hp);
      const int kvh = 2 * hp + grp;
      krs = pp_rsrc_words(p.k + ((int64_t)seg * p.k_stride + (int64_t)kvh * D) * 2, (uint32_t)T * kst_b);
      vrs = pp_rsrc_words(p.v + ((int64_t)seg * p.v_stride + (int64_t)kvh * D) * 2, (uint32_t)T * vst_b);
      dt = lo;
      dhi = hi;
    } else {
      krs[2] = 0;
      vrs[2] = 0;
      dhi = 0x7fffffff;
    }
  };
  constexpr int DMA_PARTS = 2 * S::KPW;
  const uint32_t dma_lds = gl + wg * 1024;
  auto dma_part = [&](int i, uint32_t st) __attribute__((always_inline)) {
    if (i < S::KPW)
      dma_b128(krs, dma_lds + st + i * 4096, (uint32_t)(dt * BN) * kst_b + kg_off[i]);
    else
      dma_b128(vrs, dma_lds + S::VOFF + st + (i - S::KPW) * 4096,
               (uint32_t)(dt * BN) * vst_b + vg_off[i - S::KPW]);
  };
  auto dma_advance = [&]() __attribute__((always_inline)) {
    if (__builtin_expect(++dt == dhi, 0)) dma_unit(++du);
  };
  auto dma_tile = [&](uint32_t st) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < DMA_PARTS; ++i) dma_part(i, st);
    dma_advance();
  };

  // ---- compute cursor: the unit whose tiles this wave's phases process ----
  int cu = 0;
  int seg = 0, T = 0, lo_t = 0, hi_t = 0, r0 = 0, rlast = 0, head = 0;
  int f_lo = 0, f_n = 0;     // tiles f_lo .. f_lo + f_n - 1 need no mask for this wave's rows
  bool active = false;
  __amdgpu_buffer_rsrc_t qrs;
  auto set_unit = [&](int u) __attribute__((always_inline)) {
    int q0, hp;
    unit(u, seg, T, q0, lo_t, hi_t, hp);
    head = 2 * hp + grp;
    r0 = q0 + wg * 32;
    active = r0 < T;
    rlast = min(r0 + 31, T - 1);
    int e = T;
    if (causal) e = min(e, r0 + 1);
    if (window >= 0) e = min(e, r0 + window + 1);
    const int f_hi = active ? e / BN : 0;
    f_lo = window >= 0 ? (max(0, rlast - window) + BN - 1) / BN : 0;
    f_n = max(0, f_hi - f_lo);
    qrs = pp_rsrc(p.q + ((int64_t)seg * p.q_stride + (int64_t)head * D) * 2, (uint32_t)T * qst_b);
  };
  u32x4 qreg[KST];
  // Q^T operand of the current unit (rows past the text load as zero).
  auto load_q = [&]() __attribute__((always_inline)) {
    const uint32_t qrow_b = (uint32_t)(r0 + lq) * qst_b;
#pragma unroll
    for (int i = 0; i < KST; ++i)
      qreg[i] = __builtin_amdgcn_raw_buffer_load_b128(qrs, qrow_b + (2 * i + hf) * 16, 0, 0);
  };
  // Q^T operand of unit u, loaded while the current unit's state stays in
  // place (its last softmax still needs it). Issued from inline asm like the
  // K/V loads, so the compiler tracks none of the loop's global loads; the
  // wait at the end of the softmax phase takes qreg as operands, so no use
  // of qreg can move ahead of it.
  auto load_q_of = [&](int u) __attribute__((always_inline)) {
    int sg, tn, q0, lo, hi, hp;
    unit(u, sg, tn, q0, lo, hi, hp);
    const int hd = 2 * hp + grp;
    const i32x4 rs = pp_rsrc_words(p.q + ((int64_t)sg * p.q_stride + (int64_t)hd * D) * 2, (uint32_t)tn * qst_b);
    const uint32_t qa = (uint32_t)(q0 + wg * 32 + lq) * qst_b + hf * 16;
#pragma unroll
    for (int i = 0; i < KST; ++i)
      asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen offset:%3"
                   : "=v"(qreg[i]) : "v"(qa), "s"(rs), "n"(32 * i) : "memory");
  };

  // ---- prologue: tiles 0 and 1 of both groups' streams in flight, unit 0's Q ----
  // The compiler-visible wait for the Q loads also retires tile 0's loads;
  // after it the compiler tracks no outstanding global loads, so it inserts
  // no waits of its own into the loop.
  dma_unit(0);
  set_unit(0);
  dma_tile(0);
  load_q();
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  dma_tile(S::TILE);
  lds_barrier();

  f32x16 oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[i][r] = 0.f;
  float m_i = -INFINITY;
  float l_i = 0.f;
  f32x16 sacc[NKB];
  u32x4 pk[PKS];
#pragma unroll
  for (int ks = 0; ks < PKS; ++ks)
#pragma unroll
    for (int e = 0; e < 4; ++e) pk[ks][e] = 0u;

  const float c2 = p.scale_log2;

  auto vfrag = [&](uint32_t sv, int ks, f16x8* dst) __attribute__((always_inline)) {
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
      const uint32_t vp = va[db] + sv + ks * 16 * S::ROW;
      s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(size_t)vp);
      s16x4 a2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) s16x4*)(size_t)(vp + 8 * S::ROW));
      f16x4 h1 = __builtin_bit_cast(f16x4, a1), h2 = __builtin_bit_cast(f16x4, a2);
      dst[db] = (f16x8){h1[0], h1[1], h1[2], h1[3], h2[0], h2[1], h2[2], h2[3]};
    }
  };
  auto kfrag = [&](uint32_t sk, int st, u32x4* dst) __attribute__((always_inline)) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) dst[kb] = lds_load<u32x4>(ka[st] + sk + kb * 32 * S::ROW);
  };
  // S^T = K Q^T with kr[0], kr[1] already holding the fragments of steps 0, 1;
  // `mid()` runs after the MFMAs of step KST / 2.
  auto qk_body = [&](uint32_t sK, u32x4 (*kr)[NKB], auto&& mid) __attribute__((always_inline)) {
    const f32x16 zero = {};
#pragma unroll
    for (int st = 0; st < KST; ++st) {
      if (st == KST / 2) {
        mid();
        __builtin_amdgcn_sched_barrier(0);
      }
      if (st + 2 < KST) kfrag(sK, st + 2, kr[(st + 2) % 3]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kr[st % 3][kb]),
                                                           __builtin_bit_cast(bf16x8, qreg[st]),
                                                           st == 0 ? zero : sacc[kb], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // In-place bf16 -> fp16 of this wave's slice of the V stage.
  auto conv_read = [&](uint32_t sv, u32x4* w) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < S::KPW; ++i) w[i] = lds_load<u32x4>(cv_a[i] + sv);
  };
  auto conv_write = [&](uint32_t sv, const u32x4* w) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < S::KPW; ++i) {
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        f32x2 x = {__builtin_bit_cast(float, w[i][e] << 16), __builtin_bit_cast(float, w[i][e] & 0xffff0000u)};
        o[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2));
      }
      lds_store<u32x4>(cv_a[i] + sv, o);
    }
  };

  // Output of the unit whose O^T is accumulating, captured when the compute
  // cursor leaves the unit and stored after the unit's last PV, through a
  // buffer descriptor that ends at the text's last row (the hardware drops
  // the rows past it).
  __amdgpu_buffer_rsrc_t ors;
  uint32_t o_off = 0;
  const uint32_t ost_b = (uint32_t)(p.o_stride * osz);
  auto capture_out = [&]() __attribute__((always_inline)) {
    ors = pp_rsrc(p.o + ((int64_t)seg * p.o_stride + (int64_t)head * D) * osz, (uint32_t)T * ost_b);
    // bf16: row lane / 8 (+ 8 j), 16-byte chunk lane % 8 of the 128-byte
    // row; f32: this lane's query row, first column 16 bytes * hf.
    o_off = p.out_bf16 ? (uint32_t)(r0 + (lane >> 3)) * ost_b + 16 * (lane & 7)
                       : (uint32_t)(r0 + lq) * ost_b + 16 * hf;
  };
  // O^T element (db, 4 g + e) of lane (lq, hf) is output column
  // db * 32 + 8 g + 4 hf + e. For bf16, one v_permlane32_swap per register
  // pair gives lane hf columns 16 q + 8 hf .. + 7 of 16-column group q
  // (chunk 2 q + hf of the row); the wave then transposes its 32 rows
  // through LDS (chunk c of row r at r * 128 + ((c ^ (r & 7)) << 4)), so
  // that each store writes 8 whole rows. `stg`: 4 KB of LDS that no other
  // wave touches during this phase.
  // The stores are non-temporal (nt): nothing in the launch reads O.
  auto store_out = [&](uint32_t stg) __attribute__((always_inline)) {
    const float l_tot = half_sum(l_i);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (p.out_bf16) {
      const uint32_t wr = stg + lq * 128;
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int gp = 0; gp < 2; ++gp) {
          uint32_t w[4];
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const f32x2 x = {oacc[db][8 * gp + 2 * h] * inv, oacc[db][8 * gp + 2 * h + 1] * inv};
            w[h] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2));
          }
          swap_lanes_32(w[0], w[2]);
          swap_lanes_32(w[1], w[3]);
          lds_store<u32x4>(wr + (((4 * db + 2 * gp + hf) ^ (lq & 7)) << 4), (u32x4){w[0], w[1], w[2], w[3]});
        }
      const uint32_t rrow = lane >> 3;
      const uint32_t rd = stg + rrow * 128 + (((lane & 7) ^ (rrow & 7)) << 4);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(lds_load<u32x4>(rd + j * 8 * 128), ors, o_off + j * 8 * ost_b, 0, 2);
    } else {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          u32x4 val;
#pragma unroll
          for (int e = 0; e < 4; ++e) val[e] = __builtin_bit_cast(uint32_t, oacc[db][4 * g + e] * inv);
          __builtin_amdgcn_raw_buffer_store_b128(val, ors, o_off + (db * 32 + 8 * g) * 4, 0, 2);
        }
    }
    // Zero the accumulators on the matrix core, idle during the store:
    // 0 * 0 + 0 per element, one instruction per 16 registers.
    f16x8 z = {};
#pragma unroll
    for (int i = 0; i < NDB; ++i) {
      asm volatile("" : "+v"(z));   // one opaque operand per product, so none is merged with another
      oacc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(z, z, (f32x16){}, 0, 0, 0);
    }
    m_i = -INFINITY;
    l_i = 0.f;
  };

  // ---- MFMA phase of the stream step whose K and V are in stage `st` ----
  // O^T += V^T P^T of the previous step (stage st - 1), S^T = K Q^T of this
  // step, the conversion of this wave's slice of this step's V, and at the
  // end the store of a finished unit's output (fin). LAST: the step after
  // the stream's end, PV and store only.
  bool fin = false;
  auto mphase = [&](auto last_tag, uint32_t st) __attribute__((always_inline)) {
    constexpr bool LAST = decltype(last_tag)::value;
    // (va and cv_a already point into the V stages)
    const uint32_t sK = st;
    const uint32_t sVc = st;
    const uint32_t sV = (st + (S::STAGES - 1) * S::TILE) & (S::STAGES * S::TILE - 1);
    u32x4 w[S::KPW];
    u32x4 kr[3][NKB];
    f16x8 vs[2][NDB];
    vfrag(sV, 0, vs[0]);
    vfrag(sV, 1, vs[1]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vs[ks & 1][db], __builtin_bit_cast(f16x8, pk[ks]),
                                                          oacc[db], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      if (ks + 2 < PKS) vfrag(sV, ks + 2, vs[ks & 1]);
      if (!LAST && ks + 2 >= PKS) kfrag(sK, ks + 2 - PKS, kr[ks + 2 - PKS]);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (!LAST) conv_read(sVc, w);
    __builtin_amdgcn_sched_barrier(0);
    if (!LAST) qk_body(sK, kr, [&]() __attribute__((always_inline)) { conv_write(sVc, w); });
    if (__builtin_expect(fin, 0)) {
      // Stage st + 2 (K and V halves): its tile finished two steps ago and
      // its next load is issued in this step's softmax phase. Waves 0, 1 of
      // the group take its K half, waves 2, 3 its V half.
      const uint32_t s2 = (st + 2 * S::TILE) & (S::STAGES * S::TILE - 1);
      store_out(gl + (wg >> 1) * S::VOFF + s2 + (wg & 1) * 4096);
      fin = false;
    }
  };

  // P (fp16) and its per-lane sum over this tile, with reference max `base`.
  auto make_p = [&](float base, auto&& after_step) __attribute__((always_inline)) {
    float lt0 = 0.f, lt1 = 0.f;
#pragma unroll
    for (int ks = 0; ks < PKS; ++ks) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const float x0 = sacc[ks >> 1][8 * (ks & 1) + e];
        const float x1 = sacc[ks >> 1][8 * (ks & 1) + e + 1];
        f32x2 pr = {__builtin_amdgcn_exp2f(__builtin_fmaf(x0, c2, -base)),
                    __builtin_amdgcn_exp2f(__builtin_fmaf(x1, c2, -base))};
        const uint32_t pair = __builtin_bit_cast(uint32_t, __builtin_convertvector(pr, f16x2));
        pk[ks][e / 2] = pair;
        asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]" : "+v"(lt0) : "v"(pair));
        asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "+v"(lt1) : "v"(pair));
      }
      after_step(ks);
    }
    return lt0 + lt1;
  };
  // lo <= c <= hi as one unsigned comparison (see attn_pp.hip).
  auto apply_mask = [&](int j) __attribute__((always_inline)) {
    const int kbase = j * BN + 4 * hf;
    const int dT = T - kbase;
    const int dq = r0 + lq - kbase;
    int hi = min(causal ? dq : 0x7fffffff, dT - 1);
    int lo = 0;
    if (window >= 0) {
      hi = min(hi, dq + window);
      lo = max(0, dq - window);
    }
    const bool none = hi < lo;
    const uint32_t span = none ? 0u : (uint32_t)(hi - lo);
    lo = none ? (1 << 30) : lo;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int c = kb * 32 + 8 * (r >> 2) + (r & 3);
        sacc[kb][r] = (uint32_t)(c - lo) <= span ? sacc[kb][r] : -INFINITY;
      }
  };

  // ---- softmax phase of tile t of the current unit (S^T in sacc) ----
  // The group's tile two ahead loads into stage `dst`, in parts spread over
  // the phase. On the unit's last tile the next unit's Q is loaded too and
  // the cursor moves on. At the end the wave waits for the loads it issued
  // one phase earlier. Sets `done` after the stream's last tile.
  int t = lo_t;
  bool done = false;
  auto vphase = [&](uint32_t dst) __attribute__((always_inline)) {
    if (__builtin_expect(t + 1 == hi_t && cu + 1 < nu, 0)) load_q_of(cu + 1);
    dma_part(0, dst);
    __builtin_amdgcn_sched_barrier(0);
    if (__builtin_expect((uint32_t)(t - f_lo) >= (uint32_t)f_n, 0)) apply_mask(t);
    auto mx2 = [](float a, float b) __attribute__((always_inline)) { return __builtin_elementwise_maximum(a, b); };
    float ch[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int kb = c >> 1, o = 8 * (c & 1);
      float m = mx2(sacc[kb][o], sacc[kb][o + 1]);
      m = mx2(mx2(m, sacc[kb][o + 2]), sacc[kb][o + 3]);
      m = mx2(mx2(m, sacc[kb][o + 4]), sacc[kb][o + 5]);
      ch[c] = mx2(mx2(m, sacc[kb][o + 6]), sacc[kb][o + 7]);
    }
    float mx = mx2(mx2(mx2(ch[0], ch[1]), ch[2]), ch[3]);
    mx = half_max(mx) * c2;
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(mx > m_i + 8.0f) != 0, 0)) {
      const float m_new = __builtin_elementwise_maximum(m_i, mx);
      const float alpha = m_i == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_i - m_new);
      // A row whose m_i is -inf has accumulated nothing (its O^T is zero), so
      // when no row has, scaling by alpha = 0 would change nothing: the first
      // tile of every unit skips it.
      const bool fresh = __builtin_amdgcn_ballot_w64(m_i != -INFINITY) == 0;
      m_i = m_new;
      l_i *= alpha;
      if (!fresh) {
#pragma unroll
        for (int i = 0; i < NDB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[i][r] *= alpha;
      }
    }
    l_i += make_p(m_i == -INFINITY ? 0.f : m_i, [&](int ks) __attribute__((always_inline)) {
      if (ks + 1 < DMA_PARTS) {
        __builtin_amdgcn_sched_barrier(0);
        dma_part(ks + 1, dst);
        __builtin_amdgcn_sched_barrier(0);
      }
    });
#pragma unroll
    for (int i = PKS + 1; i < DMA_PARTS; ++i) dma_part(i, dst);
    __builtin_amdgcn_sched_barrier(0);
    dma_advance();
    if (__builtin_expect(t + 1 == hi_t, 0)) {
      capture_out();
      fin = true;
      if (cu + 1 < nu) {
        set_unit(++cu);
        t = lo_t - 1;
      } else {
        done = true;
      }
    }
    ++t;
    // With at most 2 * KPW ops in flight, every load older than this phase's
    // K/V loads (the Q loads among them) is done: loads retire from vmcnt in
    // issue order. (So do stores, in one order with the loads: the stores of
    // this step's MFMA phase are done too.) This one asm statement is the
    // only wait tied to qreg: copies of qreg that the compiler placed before
    // it would read registers still in flight.
    static_assert(KST == 4, "the wait below names four Q registers");
    asm volatile("s_waitcnt vmcnt(%4)"
                 : "+v"(qreg[0]), "+v"(qreg[1]), "+v"(qreg[2]), "+v"(qreg[3])
                 : "n"(2 * S::KPW) : "memory");
  };

  // ---- the stream, in barrier-separated half-slots ----
  // Group 0: M(0) V(0) M(1) V(1) ... M(end) and one empty half-slot; group 1
  // starts with an empty half-slot and ends with M(end). The loop is unrolled
  // over the 4 stages so that every LDS stage offset is an immediate.
  auto step = [&](auto stage_tag) __attribute__((always_inline)) {
    constexpr uint32_t SI = decltype(stage_tag)::value;
    mphase(std::false_type{}, SI * S::TILE);
    lds_barrier();
    vphase(((SI + 2) & 3) * S::TILE);
    lds_barrier();
    return !done;
  };
  if (grp) lds_barrier();
  uint32_t end_st;
  for (;;) {
    if (!step(std::integral_constant<uint32_t, 0>{})) { end_st = 1; break; }
    if (!step(std::integral_constant<uint32_t, 1>{})) { end_st = 2; break; }
    if (!step(std::integral_constant<uint32_t, 2>{})) { end_st = 3; break; }
    if (!step(std::integral_constant<uint32_t, 3>{})) { end_st = 0; break; }
  }
  mphase(std::true_type{}, end_st * S::TILE);
  // Loads past the stream's end may still be writing LDS.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  lds_barrier();
  if (!grp) lds_barrier();
}

}  // namespace

bool bf16_pp64_kernel(int d, AttnKernelFn* fn, int* bn, int* nw, int* lds) {
  switch (d) {
    case 64: *fn = attn_pp64_kernel<64>; *bn = 64; *nw = 8; *lds = PP64Shape<64>::LDS; return true;
    default: return false;
  }
}

}  // namespace inl
