// Persistent bf16 attention for head_dim 256 on gfx950.
//
// Same schedule, masks and results as the other attention kernels (per-wave
// math as in attn_fwd.hip: S^T = K.Q^T on bf16 MFMA, lane-local softmax on
// query columns, O^T += V^T.P^T on fp16 MFMA with P rounded to fp16 and the
// row sum taken over the rounded values). At head_dim 256 a wave's O^T alone
// is 128 VGPRs and Q^T another 64, so two waves per SIMD do not fit; this
// kernel runs one wave per SIMD with the whole 512-register file and
// overlaps the softmax with the matrix core inside each wave:
//
//   - A workgroup is 4 waves, one per SIMD, on one CU, walking the same
//     host-built stream of work units as attn_pp.hip. Each wave owns 32
//     query rows of one head; a unit is hpw heads x 4 / hpw blocks of rows.
//   - Tiles are 32 keys. Iteration j computes P of tile j's first 16 keys
//     in the shadow of S^T = K Q^T of tile j + 1 (S^T double-buffered), P of
//     its other 16 keys beside O^T += V^T P^T of the first 16, and the
//     bf16 -> fp16 conversion of the wave's slice of V_{j+1} beside the PV
//     of the second 16; then it issues the loads of tile j + 3. The row sum
//     of P is one more MFMA per 16 keys, with an all-ones A operand.
//   - 4 LDS stages of K (bf16) and V (fp16 after conversion), 16 KiB each;
//     one barrier per tile.
//
// LDS layout (per stage, rows of 256 bf16 / fp16 = 512 bytes):
//   K: 16-byte chunk c of key row r at r * 512 + ((c ^ (r & 15)) * 16).
//   V: chunk c of row r at r * 512 + ((c ^ ((r & 3) << 2)) * 16).
// As in attn_pp.hip, both swizzles are applied by choosing which global
// chunk each lane loads, and V is converted in place.

#include <type_traits>

#include "attn_stream.hpp"

namespace inl {

namespace {

template <int D, int BN>
struct WideShape {
  static_assert(PP_MAX_UNITS % 4 == 0, "descriptor table alignment");
  static constexpr int NW = 4;              // waves, one per SIMD
  static constexpr int NT = NW * 64;
  static constexpr int CH = D / 8;          // 16-byte chunks per row
  static constexpr int ROW = D * 2;         // bytes per K or V row in LDS
  static constexpr int TILE = BN * ROW;     // bytes per stage
  static constexpr int STAGES = 4;
  static constexpr int TILES_LDS = 2 * STAGES * TILE;
  static constexpr int LDS = TILES_LDS + PP_MAX_UNITS * (16 + 4);
  static constexpr int KPW = TILE / 1024 / NW;  // 1 KB direct loads per wave per tile (K and V each)
  static constexpr int RPB = 1024 / ROW;        // rows per 1 KB block
  static_assert(D == 256 && BN == 32, "laid out for 32 chunks per row and one 32-key block");
  static_assert(KPW >= 1 && RPB >= 1, "tile shape");
};

template <int D, int BN>
__global__ __launch_bounds__(256, 1) void attn_wide_kernel(AttnParams p) {
  using S = WideShape<D, BN>;
  constexpr int NDB = D / 32;    // 32-wide d blocks of O^T
  constexpr int KST = D / 16;    // k-steps of the QK^T product
  constexpr int PKS = BN / 16;   // k-steps of the PV product

  extern __shared__ __attribute__((aligned(16))) char smem[];
  const uint32_t lds0 = lds_addr(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31;
  const int hf = lane >> 5;

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
  __syncthreads();

  const int causal = p.causal;
  const int window = p.window;
  const uint32_t kst_b = (uint32_t)(p.k_stride * 2);
  const uint32_t vst_b = (uint32_t)(p.v_stride * 2);
  const uint32_t qst_b = (uint32_t)(p.q_stride * 2);
  const int osz = p.out_bf16 ? 2 : 4;

  auto unit = [&](int u, int& seg, int& T, int& q0, int& lo, int& hi, int& hg) __attribute__((always_inline)) {
    const int4 d = sdesc[u];
    seg = __builtin_amdgcn_readfirstlane(d.x);
    T = __builtin_amdgcn_readfirstlane(d.y);
    q0 = __builtin_amdgcn_readfirstlane(d.z);
    lo = (int)((uint32_t)__builtin_amdgcn_readfirstlane(d.w) >> 16);
    hi = __builtin_amdgcn_readfirstlane(d.w) & 0xffff;
    hg = __builtin_amdgcn_readfirstlane(shg[u]);
  };

  // ---- per-lane constants ----
  // This wave's slice of every tile: 1 KB blocks i * NW + wave.
  uint32_t kg_off[S::KPW], vg_off[S::KPW];
  uint32_t cv_a[S::KPW];   // LDS address of the stage-0 V chunk this lane converts
#pragma unroll
  for (int i = 0; i < S::KPW; ++i) {
    const int blk = i * S::NW + wave;
    const int row = blk * S::RPB + lane / S::CH;
    const int pc = lane % S::CH;
    kg_off[i] = (uint32_t)row * kst_b + ((pc ^ (row & 15)) << 4);
    vg_off[i] = (uint32_t)row * vst_b + ((pc ^ ((row & 3) << 2)) << 4);
    cv_a[i] = opaque(lds0 + S::STAGES * S::TILE + blk * 1024 + lane * 16);
  }
  uint32_t ka[KST];   // QK^T fragment of step st (rows lq of the 32-key block), stage 0
#pragma unroll
  for (int st = 0; st < KST; ++st) ka[st] = opaque(lds0 + lq * S::ROW + (((2 * st + hf) ^ (lq & 15)) << 4));
  const int g16 = lane >> 4;
  const int j16 = lane & 15;
  const int vcol = 16 * (g16 & 1) + 4 * (j16 & 3);
  const int vrow = 4 * hf + (j16 >> 2);
  uint32_t va[NDB];   // PV fragment of d block db (rows vrow, vrow + 8 of a k-step), stage 0
#pragma unroll
  for (int db = 0; db < NDB; ++db)
    va[db] = opaque(lds0 + S::STAGES * S::TILE + vrow * S::ROW +
                    ((((4 * db + (vcol >> 3)) ^ ((vrow & 3) << 2)) << 4) | ((vcol * 2) & 15)));

  // ---- load cursor: the next tile of the stream to load (stage = index % 4) ----
  // Past the stream's end the descriptors get an empty range: the loads go
  // out without a branch and return zeros into a stage no later phase reads.
  int du = 0, dt = 0, dhi = 0;
  i32x4 krs, vrs;
  auto dma_unit = [&](int u) __attribute__((always_inline)) {
    if (u < nu) {
      int seg, T, q0, lo, hi, hg;
      unit(u, seg, T, q0, lo, hi, hg);
      const int kvh = hg / p.groups_per_kv;
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
  const uint32_t dma_lds = lds0 + wave * 1024;
  auto dma_part = [&](int i, uint32_t st) __attribute__((always_inline)) {
    if (i < S::KPW)
      dma_b128(krs, dma_lds + st + i * (S::NW * 1024), (uint32_t)(dt * BN) * kst_b + kg_off[i]);
    else
      dma_b128(vrs, dma_lds + S::STAGES * S::TILE + st + (i - S::KPW) * (S::NW * 1024),
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

  // ---- softmax / PV cursor: the unit of tile j ----
  int cu = 0;
  int seg = 0, T = 0, lo_t = 0, hi_t = 0, r0 = 0, rlast = 0, head = 0;
  int f_lo = 0, f_n = 0;     // tiles f_lo .. f_lo + f_n - 1 need no mask for this wave's rows
  bool active = false;
  __amdgpu_buffer_rsrc_t qrs;
  auto set_unit = [&](int u) __attribute__((always_inline)) {
    int q0, hg;
    unit(u, seg, T, q0, lo_t, hi_t, hg);
    const int kvh = hg / p.groups_per_kv;
    head = kvh * p.group + (hg - kvh * p.groups_per_kv) * p.hpw + wave / p.rb;
    r0 = q0 + (wave % p.rb) * 32;
    active = r0 < T;
    rlast = min(r0 + 31, T - 1);
    // Tile j needs no mask iff j * BN + BN <= e and j * BN >= b (see
    // apply_mask).
    int e = T;
    if (causal) e = min(e, r0 + 1);
    if (window >= 0) e = min(e, r0 + window + 1);
    const int f_hi = active ? e / BN : 0;
    f_lo = window >= 0 ? (max(0, rlast - window) + BN - 1) / BN : 0;
    f_n = max(0, f_hi - f_lo);
    qrs = pp_rsrc(p.q + ((int64_t)seg * p.q_stride + (int64_t)head * D) * 2, (uint32_t)T * qst_b);
  };
  // ---- QK cursor: the unit of tile j + 1 (its last tile triggers the next Q load) ----
  int qu = 0, qt = 0, qhi = 0;

  u32x4 qreg[KST];
  auto load_q = [&]() __attribute__((always_inline)) {
    const uint32_t qrow_b = (uint32_t)(r0 + lq) * qst_b;
#pragma unroll
    for (int i = 0; i < KST; ++i)
      qreg[i] = __builtin_amdgcn_raw_buffer_load_b128(qrs, qrow_b + (2 * i + hf) * 16, 0, 0);
  };
  // Q^T of unit u, loaded into qreg once the current unit's last QK^T has
  // read it. The 16 loads and a full wait form ONE asm statement, so every
  // value is complete before the compiler can use or copy it: with ~450
  // registers live it moves Q^T between VGPRs and AGPRs, and a copy of a
  // register whose load is still in flight would take stale data (which is
  // what a load-now, wait-later form produced). The outputs are AGPRs, where
  // the allocator keeps Q^T as the QK^T MFMAs' B operand. The wait also
  // retires the K/V loads issued before it; it stalls once per unit.
  auto load_q_of = [&](int u) __attribute__((always_inline)) {
    int sg, tn, q0, lo, hi, hg;
    unit(u, sg, tn, q0, lo, hi, hg);
    const int kvh = hg / p.groups_per_kv;
    const int hd = kvh * p.group + (hg - kvh * p.groups_per_kv) * p.hpw + wave / p.rb;
    const i32x4 rs = pp_rsrc_words(p.q + ((int64_t)sg * p.q_stride + (int64_t)hd * D) * 2, (uint32_t)tn * qst_b);
    const uint32_t qa = (uint32_t)(q0 + (wave % p.rb) * 32 + lq) * qst_b + hf * 16;
    static_assert(KST == 16, "the asm below loads sixteen Q registers");
    asm volatile(
        "buffer_load_dwordx4 %0, %16, %17, 0 offen offset:0\n\t"
        "buffer_load_dwordx4 %1, %16, %17, 0 offen offset:32\n\t"
        "buffer_load_dwordx4 %2, %16, %17, 0 offen offset:64\n\t"
        "buffer_load_dwordx4 %3, %16, %17, 0 offen offset:96\n\t"
        "buffer_load_dwordx4 %4, %16, %17, 0 offen offset:128\n\t"
        "buffer_load_dwordx4 %5, %16, %17, 0 offen offset:160\n\t"
        "buffer_load_dwordx4 %6, %16, %17, 0 offen offset:192\n\t"
        "buffer_load_dwordx4 %7, %16, %17, 0 offen offset:224\n\t"
        "buffer_load_dwordx4 %8, %16, %17, 0 offen offset:256\n\t"
        "buffer_load_dwordx4 %9, %16, %17, 0 offen offset:288\n\t"
        "buffer_load_dwordx4 %10, %16, %17, 0 offen offset:320\n\t"
        "buffer_load_dwordx4 %11, %16, %17, 0 offen offset:352\n\t"
        "buffer_load_dwordx4 %12, %16, %17, 0 offen offset:384\n\t"
        "buffer_load_dwordx4 %13, %16, %17, 0 offen offset:416\n\t"
        "buffer_load_dwordx4 %14, %16, %17, 0 offen offset:448\n\t"
        "buffer_load_dwordx4 %15, %16, %17, 0 offen offset:480\n\t"
        "s_waitcnt vmcnt(0)"
        : "=&a"(qreg[0]), "=&a"(qreg[1]), "=&a"(qreg[2]), "=&a"(qreg[3]), "=&a"(qreg[4]), "=&a"(qreg[5]),
          "=&a"(qreg[6]), "=&a"(qreg[7]), "=&a"(qreg[8]), "=&a"(qreg[9]), "=&a"(qreg[10]), "=&a"(qreg[11]),
          "=&a"(qreg[12]), "=&a"(qreg[13]), "=&a"(qreg[14]), "=&a"(qreg[15])
        : "v"(qa), "s"(rs)
        : "memory");
  };
  auto wait_loads = [&]() __attribute__((always_inline)) {
    // all but this iteration's K/V loads
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(DMA_PARTS) : "memory");
  };

  f32x16 oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[i][r] = 0.f;
  float m_i = -INFINITY;
  float l_i = 0.f;   // row sum of the rounded fp16 P (whole row in every lane)
  f32x16 sacc[2];    // S^T of tiles j (sacc[j & 1]) and j + 1
  u32x4 pk[PKS];     // P^T operand per PV k-step
  const float c2 = p.scale_log2;

  auto kfrag = [&](uint32_t sk, int st) __attribute__((always_inline)) {
    return lds_load<u32x4>(ka[st] + sk);
  };
  auto vfrag = [&](uint32_t sv, int ks, int db) __attribute__((always_inline)) {
    const uint32_t vp = va[db] + sv + ks * 16 * S::ROW;
    s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(size_t)vp);
    s16x4 a2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4*)(size_t)(vp + 8 * S::ROW));
    f16x4 h1 = __builtin_bit_cast(f16x4, a1), h2 = __builtin_bit_cast(f16x4, a2);
    return (f16x8){h1[0], h1[1], h1[2], h1[3], h2[0], h2[1], h2[2], h2[3]};
  };
  auto conv = [&](uint32_t sv) __attribute__((always_inline)) {
    u32x4 w[S::KPW];
#pragma unroll
    for (int i = 0; i < S::KPW; ++i) w[i] = lds_load<u32x4>(cv_a[i] + sv);
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
  // S^T = K Q^T of the tile in stage `sk` into acc (prologue only; the loop
  // interleaves the same reads and MFMAs with the softmax).
  auto qk = [&](uint32_t sk, f32x16& acc) __attribute__((always_inline)) {
    u32x4 kr[KST];
#pragma unroll
    for (int st = 0; st < KST; ++st) kr[st] = kfrag(sk, st);
    const f32x16 zero = {};
#pragma unroll
    for (int st = 0; st < KST; ++st)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kr[st]),
                                                    __builtin_bit_cast(bf16x8, qreg[st]), st == 0 ? zero : acc, 0, 0, 0);
  };

  // Key of element r is kbase + c with c a compile-time offset. lo <= c <= hi
  // (lo: the window of the last row; hi: the text end, the causal diagonal
  // and the window of the first row) as one unsigned comparison,
  // c - lo <= hi - lo; an empty range becomes lo = 2^30, where c - lo wraps
  // above any span. Without a window lo = 0 (c >= 0 anyway).
  auto apply_mask = [&](f32x16& s, int j) __attribute__((always_inline)) {
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
    for (int r = 0; r < 16; ++r) {
      const int c = 8 * (r >> 2) + (r & 3);
      s[r] = (uint32_t)(c - lo) <= span ? s[r] : -INFINITY;
    }
  };

  // The stores go through a buffer descriptor that ends at the text's last
  // row, so the hardware drops the rows past it without a branch.
  __amdgpu_buffer_rsrc_t ors;
  uint32_t o_off = 0;
  const uint32_t ost_b = (uint32_t)(p.o_stride * osz);
  auto capture_out = [&]() __attribute__((always_inline)) {
    ors = pp_rsrc(p.o + ((int64_t)seg * p.o_stride + (int64_t)head * D) * osz, (uint32_t)T * ost_b);
    // bf16: row lane / 8 (+ 8 j), 16-byte chunk lane % 8 of a 128-byte
    // quarter row; f32: this lane's query row, first column 16 bytes * hf.
    o_off = p.out_bf16 ? (uint32_t)(r0 + (lane >> 3)) * ost_b + 16 * (lane & 7)
                       : (uint32_t)(r0 + lq) * ost_b + 16 * hf;
  };
  // O^T element (db, 4 g + e) of lane (lq, hf) is output column
  // db * 32 + 8 g + 4 hf + e. For bf16, one v_permlane32_swap per register
  // pair gives lane hf = 0 columns 16 q .. 16 q + 7 and lane hf = 1 columns
  // 16 q + 8 .. 16 q + 15 (16 contiguous bytes, chunk 2 q + hf of the row).
  // The wave then transposes its 32 rows through LDS, one 128-byte quarter
  // row at a time (chunk c of row r at r * 128 + ((c ^ (r & 7)) << 4)), so
  // that each store writes 8 whole 128-byte lines. `stg`: 4 KB of LDS that
  // no other wave touches during this step.
  // The stores are non-temporal (nt): nothing in the launch reads O.
  auto store_out = [&](uint32_t stg) __attribute__((always_inline)) {
    const float l_tot = l_i;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (p.out_bf16) {
      const uint32_t wr = stg + lq * 128;
      const uint32_t rrow = lane >> 3;
      const uint32_t rd = stg + rrow * 128 + (((lane & 7) ^ (rrow & 7)) << 4);
#pragma unroll
      for (int part = 0; part < NDB / 2; ++part) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int db = 2 * part + (i >> 1), gp = i & 1;
          uint32_t w[4];
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const f32x2 x = {oacc[db][8 * gp + 2 * h] * inv, oacc[db][8 * gp + 2 * h + 1] * inv};
            w[h] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, bf16x2));
          }
          swap_lanes_32(w[0], w[2]);
          swap_lanes_32(w[1], w[3]);
          lds_store<u32x4>(wr + (((2 * i + hf) ^ (lq & 7)) << 4), (u32x4){w[0], w[1], w[2], w[3]});
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
          __builtin_amdgcn_raw_buffer_store_b128(lds_load<u32x4>(rd + j * 8 * 128), ors,
                                                 o_off + j * 8 * ost_b + part * 128, 0, 2);
      }
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

  // ---- prologue: tiles 0, 1 resident, tile 2 in flight, S^T of tile 0 ----
  dma_unit(0);
  set_unit(0);
  qu = 0;
  qt = lo_t;
  qhi = hi_t;
  dma_tile(0);
  dma_tile(S::TILE);
  load_q();
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): tiles 0, 1 and Q
  lds_barrier();                       // every wave's slice of tiles 0, 1
  conv(0);
  qk(0, sacc[0]);
  // The QK cursor moves to tile 1; if tile 0 ended its unit, the next Q.
  if (qt + 1 == qhi && qu + 1 < nu) load_q_of(qu + 1);
  if (++qt == qhi && ++qu < nu) {
    int a, b, c, lo, hi, d;
    unit(qu, a, b, c, lo, hi, d);
    qt = lo;
    qhi = hi;
  }
  dma_tile(2 * S::TILE);
  wait_loads();
  lds_barrier();

  // ---- the stream, one barrier per tile ----
  // Iteration j: softmax of tile j (stage j % 4, S^T in sacc[j & 1]) beside
  // QK^T of tile j + 1; PV of tile j beside the conversion of tile j + 1's
  // V and the loads of tile j + 3; the store when tile j ends its unit.
  int t = lo_t;
  bool done = false;
  auto step = [&](auto stage_tag) __attribute__((always_inline)) {
    constexpr uint32_t SI = decltype(stage_tag)::value;
    constexpr uint32_t st_cur = SI * S::TILE;
    constexpr uint32_t st_nxt = ((SI + 1) & 3) * S::TILE;
    constexpr uint32_t st_dma = ((SI + 3) & 3) * S::TILE;
    f32x16& s_cur = sacc[SI & 1];
    f32x16& s_nxt = sacc[(SI + 1) & 1];

    // softmax of tile j: mask, row max, lazy rescale
    if (__builtin_expect((uint32_t)(t - f_lo) >= (uint32_t)f_n, 0)) apply_mask(s_cur, t);
    float mx;
    {
      auto mx2 = [](float a, float b) __attribute__((always_inline)) { return __builtin_elementwise_maximum(a, b); };
      float c0 = mx2(s_cur[0], s_cur[1]), c1 = mx2(s_cur[2], s_cur[3]);
      c0 = mx2(mx2(c0, s_cur[4]), s_cur[5]);
      c1 = mx2(mx2(c1, s_cur[6]), s_cur[7]);
      c0 = mx2(mx2(c0, s_cur[8]), s_cur[9]);
      c1 = mx2(mx2(c1, s_cur[10]), s_cur[11]);
      c0 = mx2(mx2(c0, s_cur[12]), s_cur[13]);
      c1 = mx2(mx2(c1, s_cur[14]), s_cur[15]);
      mx = half_max(mx2(c0, c1)) * c2;
    }
    if (__builtin_expect(__builtin_amdgcn_ballot_w64(mx > m_i + 8.0f) != 0, 0)) {
      const float m_new = __builtin_elementwise_maximum(m_i, mx);
      const float alpha = m_i == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_i - m_new);
      // A row whose m_i is -inf has accumulated nothing (its O^T is zero), so
      // when no row has, scaling by alpha = 0 would change nothing: the first
      // tile of every unit skips it.
      const bool fresh = __builtin_amdgcn_ballot_w64(m_i != -INFINITY) == 0;
      m_i = m_new;
      l_i *= alpha;
      // O^T lives in AGPRs (the PV MFMAs' accumulators); the products go
      // back there explicitly, so that the paths with and without this
      // rescale meet in AGPRs instead of copying O^T through VGPRs.
      if (!fresh) {
#pragma unroll
        for (int i = 0; i < NDB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            float y;
            asm("v_accvgpr_write_b32 %0, %1" : "=a"(y) : "v"(oacc[i][r] * alpha));
            oacc[i][r] = y;
          }
      }
    }
    // Three MFMA groups, each with VALU and LDS work in its shadow:
    //   QK^T of tile j + 1 (16)   P of k-step 0, its V fragments, K reads
    //   PV k-step 0 (8 + 1)       P of k-step 1, its V fragments
    //   PV k-step 1 (8 + 1)       conversion of tile j + 1's V
    // The row sum of P comes from the matrix core: one extra MFMA per k-step
    // with an all-ones A operand sums the rounded fp16 P over the k-step's
    // keys into every row of its accumulator (f32 accumulation).
    const float base = m_i == -INFINITY ? 0.f : m_i;
    u32x4 kr[KST];
#pragma unroll
    for (int st = 0; st < KST; ++st) kr[st] = kfrag(st_nxt, st);
    f16x8 vf0[NDB], vf1[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) vf0[db] = vfrag(st_cur, 0, db);
    auto make_pk = [&](int ks) __attribute__((always_inline)) {
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        f32x2 pr = {__builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[8 * ks + e], c2, -base)),
                    __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[8 * ks + e + 1], c2, -base))};
        pk[ks][e / 2] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pr, f16x2));
      }
    };
    make_pk(0);
    {
      const f32x16 zero = {};
#pragma unroll
      for (int st = 0; st < KST; ++st)
        s_nxt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, kr[st]),
                                                        __builtin_bit_cast(bf16x8, qreg[st]),
                                                        st == 0 ? zero : s_nxt, 0, 0, 0);
    }
    // 8 K reads ahead; per QK^T MFMA one more K read, one V read (8 of 16)
    // and the VALU of P's first k-step
    __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
#pragma unroll
    for (int i = 0; i < KST; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    const f16x8 ones = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f,
                        (_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};
    f32x16 lsum;
    make_pk(1);
#pragma unroll
    for (int db = 0; db < NDB; ++db) vf1[db] = vfrag(st_cur, 1, db);
    {
      const f32x16 zero = {};
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf0[db], __builtin_bit_cast(f16x8, pk[0]), oacc[db], 0, 0, 0);
      lsum = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones, __builtin_bit_cast(f16x8, pk[0]), zero, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < NDB + 1; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 1);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    }
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int db = 0; db < NDB; ++db)
      oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf1[db], __builtin_bit_cast(f16x8, pk[1]), oacc[db], 0, 0, 0);
    lsum = __builtin_amdgcn_mfma_f32_32x32x16_f16(ones, __builtin_bit_cast(f16x8, pk[1]), lsum, 0, 0, 0);
    conv(st_nxt);
#pragma unroll
    for (int i = 0; i < NDB + 1; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 2);
    }
    __builtin_amdgcn_sched_barrier(0);
    // The next unit's Q once the current one's last QK^T has run (its wait
    // retires the loads issued before it, not this step's), then the loads
    // of tile j + 3: issued at the end of the step, they run faster than
    // anywhere earlier, where they share LDS with the fragment reads.
    // The QK cursor moves to tile j + 2, into the next unit (whose Q^T is
    // loaded now) when tile j + 1 ended its unit: one test for both.
    if (__builtin_expect(++qt == qhi, 0)) {
      if (qu + 1 < nu) load_q_of(qu + 1);
      if (++qu < nu) {
        int a, b, c, lo, hi, d;
        unit(qu, a, b, c, lo, hi, d);
        qt = lo;
        qhi = hi;
      }
    }
#pragma unroll
    for (int i = 0; i < DMA_PARTS; ++i) dma_part(i, st_dma);
    __builtin_amdgcn_sched_barrier(0);
    l_i += lsum[0];
    dma_advance();
    // the softmax / PV cursor moves to tile j + 1
    if (__builtin_expect(t + 1 == hi_t, 0)) {
      capture_out();
      // The K half of this step's stage: its QK^T ran in the previous step,
      // and its next load is issued in the next one.
      store_out(lds0 + st_cur + wave * 4096);
      if (cu + 1 < nu) {
        set_unit(++cu);
        t = lo_t - 1;
      } else {
        done = true;
      }
    }
    ++t;
    wait_loads();
    lds_barrier();
    return !done;
  };
  for (;;) {
    if (!step(std::integral_constant<uint32_t, 0>{})) break;
    if (!step(std::integral_constant<uint32_t, 1>{})) break;
    if (!step(std::integral_constant<uint32_t, 2>{})) break;
    if (!step(std::integral_constant<uint32_t, 3>{})) break;
  }
  // Loads past the stream's end may still be writing LDS.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  lds_barrier();
}

}  // namespace

bool bf16_wide_kernel(int d, AttnKernelFn* fn, int* bn, int* nw, int* lds) {
  switch (d) {
    case 256: *fn = attn_wide_kernel<256, 32>; *bn = 32; *nw = 4; *lds = WideShape<256, 32>::LDS; return true;
    default: return false;
  }
}

}  // namespace inl
