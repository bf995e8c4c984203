// bf16 fast path of the packed varlen attention for gfx950.
//
// Same schedule, masks and per-wave math as attn_fwd.hip's generic kernel
// (S^T = K.Q^T on bf16 MFMA, lane-local online softmax, O^T += V^T.P^T on
// fp16 MFMA), with the staging built on gfx950's data movers:
//   - K tiles go global -> LDS with `buffer_load_dwordx4 ... lds` (no VGPR
//     staging). Each lane picks the global chunk that lands on its LDS slot,
//     which writes the XOR-swizzled layout the ds_read_b128 of the S^T
//     product reads without bank conflicts.
//   - V tiles are loaded to registers (buffer loads), converted bf16 -> fp16
//     and stored row-major (rows padded by 32 bytes); the PV product reads
//     them transposed with
//     `ds_read_b64_tr_b16` (within 16 lanes, lane j receives element j % 4 of
//     the 8 bytes addressed by lanes 4e + j / 4, e = 0..3), so no transpose
//     is done by ALU instructions.
//   - Buffer resources bound every text's rows: loads past the text return
//     zero, so no load needs a branch.
// The kernel serves head_dim 64 and 256 (128 takes the ping-pong kernel in
// attn_pp.hip); other head dims take the generic kernel.

#include <type_traits>

#include "attn_kernels.hpp"

namespace inl {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  // word3 0x00020000: raw (untyped) 32-bit data, the gfx9 buffer format.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// V tiles are stored fp16, row-major, with rows padded by 32 bytes: a 16-lane
// transposed read touches 4 consecutive rows x 2 chunks, and a row pitch of
// 2 (mod 8) 16-byte units puts those 8 chunks in 8 distinct bank groups while
// every fragment offset stays linear in (ks, db).
template <int D>
constexpr int vrow_bytes() { return D * 2 + 32; }

// D = 256 needs ~300 registers (O^T alone is 128) and 136 KB of LDS, one
// workgroup per CU: it is built for one wave per SIMD.
template <int D, int BN, int NW>
__global__ __launch_bounds__(NW * 64, D >= 256 ? 1 : 2) void attn_bf16_kernel(AttnParams p) {
  constexpr int NT = NW * 64;
  constexpr int CH = D / 8;               // 16-byte chunks per row
  constexpr int ROW = D * 2;              // bytes per K or V row in LDS
  constexpr int TILE = BN * ROW;          // bytes of one K tile
  constexpr int VROWB = vrow_bytes<D>();  // bytes per V row in LDS (padded)
  constexpr int STAGE = TILE + BN * VROWB;  // K tile + V tile
  constexpr int KBLK = TILE / 1024;       // 1 KB direct-load blocks per K tile
  constexpr int KPT = KBLK / NW;          // direct loads per wave per tile
  constexpr int VPT = (BN * CH) / NT;     // V chunks per thread per tile
  constexpr int NKB = BN / 32;
  constexpr int NDB = D / 32;
  static_assert(KBLK % NW == 0 && (BN * CH) % NT == 0, "tile / wave shape");
  static_assert(CH >= 8 && 64 % CH == 0, "row shape");

  extern __shared__ __attribute__((aligned(16))) char smem[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int lq = lane & 31;
  const int hf = lane >> 5;

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
  const __amdgpu_buffer_rsrc_t krs =
      make_rsrc(p.k + ((int64_t)seg * p.k_stride + (int64_t)kvh * D) * 2, (uint32_t)T * kst_b);
  const __amdgpu_buffer_rsrc_t vrs =
      make_rsrc(p.v + ((int64_t)seg * p.v_stride + (int64_t)kvh * D) * 2, (uint32_t)T * vst_b);

  // Q^T operand in registers (rows past the text load as zero).
  const uint32_t qst_b = (uint32_t)(p.q_stride * 2);
  const __amdgpu_buffer_rsrc_t qrs =
      make_rsrc(p.q + ((int64_t)seg * p.q_stride + (int64_t)head * D) * 2, (uint32_t)T * qst_b);
  const int qrow = r0 + lq;
  u32x4 qreg[D / 16];
#pragma unroll
  for (int i = 0; i < D / 16; ++i)
    qreg[i] = __builtin_amdgcn_raw_buffer_load_b128(qrs, (uint32_t)qrow * qst_b + (2 * i + hf) * 16, 0, 0);

  f32x16 oacc[NDB];
#pragma unroll
  for (int i = 0; i < NDB; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[i][r] = 0.f;
  float m_i = -INFINITY;
  // Row sum of the rounded fp16 P, in f32 adds: v_dot2_f32_f16 would add a
  // pair per instruction but waits for the matrix core, which the other
  // waves of the SIMD keep busy.
  float l_i = 0.f;

  u32x4 vreg[VPT];

  // Issue the loads of tile t: K straight into LDS stage `buf`, V into vreg.
  auto issue = [&](int t, int buf) {
    char* sK = smem + buf * STAGE;
    const int key0 = t * BN;
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int blk = i * NW + wave;                   // 1 KB block of the tile
      const int row = blk * (64 / CH) + lane / CH;     // tile row this lane fills
      const int lc = (lane % CH) ^ (row & 7);          // logical chunk for its slot
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          krs, LDS_PTR(sK + blk * 1024), 16, (uint32_t)(key0 + row) * kst_b + lc * 16, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int id = i * NT + tid;
      const int row = id / CH, c = id % CH;
      vreg[i] = __builtin_amdgcn_raw_buffer_load_b128(vrs, (uint32_t)(key0 + row) * vst_b + c * 16, 0, 0);
    }
  };
  // Convert the V registers to fp16 and store them into stage `buf`.
  auto store_v = [&](int buf) {
    char* sV = smem + buf * STAGE + TILE;
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int id = i * NT + tid;
      const int row = id / CH, c = id % CH;
      u32x4 w = vreg[i], o;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f32x2 x = {__builtin_bit_cast(float, w[j] << 16), __builtin_bit_cast(float, w[j] & 0xffff0000u)};
        o[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(x, f16x2));
      }
      *reinterpret_cast<u32x4*>(sV + row * VROWB + c * 16) = o;
    }
  };

  if (lo_t < hi_t) {
    issue(lo_t, 0);
    store_v(0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  const float c2 = p.scale_log2;
  const int g16 = lane >> 4;        // 16-lane group of the transposed reads
  const int j16 = lane & 15;

  // Per-lane LDS byte offsets that do not change across tiles.
  int koff[D / 16];                 // K fragment of step st, row lq (+ kb*32 rows)
#pragma unroll
  for (int st = 0; st < D / 16; ++st) koff[st] = lq * ROW + (((2 * st + hf) ^ (lq & 7)) << 4);
  const int vcol = 16 * (g16 & 1) + 4 * (j16 & 3);
  const int vrow = 4 * hf + (j16 >> 2);
  // V^T fragment (db, ks, half): rows ks*16 + 8*half + vrow, columns
  // db*32 + vcol, at a linear offset from this per-lane base.
  const int vbase_off = vrow * VROWB + vcol * 2;

  for (int t = lo_t; t < hi_t; ++t) {
    const int buf = (t - lo_t) & 1;
    const bool more = t + 1 < hi_t;
    if (more) issue(t + 1, buf ^ 1);

    const int kt0 = t * BN;
    // One tile of work: S^T, optional mask, softmax, PV. Instantiated twice so
    // the common unmasked tile never merges with the masked one (no register
    // copies of the S accumulators at a join).
    auto tile = [&](auto masked) {
      constexpr bool MASK = decltype(masked)::value;
      const char* sK = smem + buf * STAGE;
      const char* sV = sK + TILE;

      // ---- S^T = K . Q^T: K fragments read one step ahead of the MFMAs ----
      f32x16 sacc[NKB];
      bf16x8 kf[NKB], kn[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        kf[kb] = *reinterpret_cast<const bf16x8*>(sK + kb * 32 * ROW + koff[0]);
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
      }
#pragma unroll
      for (int st = 0; st < D / 16; ++st) {
        if (st + 1 < D / 16) {
#pragma unroll
          for (int kb = 0; kb < NKB; ++kb)
            kn[kb] = *reinterpret_cast<const bf16x8*>(sK + kb * 32 * ROW + koff[st + 1]);
        }
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
          sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kb], __builtin_bit_cast(bf16x8, qreg[st]), sacc[kb], 0, 0, 0);
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) kf[kb] = kn[kb];
      }

      if constexpr (MASK) {
        const int qi = r0 + lq;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int kj = kt0 + kb * 32 + 8 * (r >> 2) + 4 * hf + (r & 3);
            bool ok = kj < T;
            if (p.causal) ok = ok && kj <= qi;
            if (p.window >= 0) ok = ok && abs(qi - kj) <= p.window;
            sacc[kb][r] = ok ? sacc[kb][r] : -INFINITY;
          }
      }

      // ---- row max (v_maximum3: no NaN canonicalisation), across halves ----
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

      // Lazy rescaling: the reference max moves only when a row's max grows
      // by more than 2^8 (P then stays <= 256, exact range for fp16).
      if (__builtin_amdgcn_ballot_w64(mx > m_i + 8.0f)) {
        const float m_new = __builtin_elementwise_maximum(m_i, mx);
        // m_i = -inf: nothing accumulated yet, alpha = 0 (and no -inf - -inf)
        const float alpha = __builtin_amdgcn_exp2f(m_i - (m_new == -INFINITY ? 0.f : m_new));
        m_i = m_new;
        l_i *= alpha;
#pragma unroll
        for (int i = 0; i < NDB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[i][r] *= alpha;
      }
      const float base = (m_i == -INFINITY) ? 0.f : m_i;

      // ---- P (fp16) per 16-key step, then O^T += V^T . P^T ----
      const char* vptr = sV + vbase_off;
#pragma unroll
      for (int ks = 0; ks < BN / 16; ++ks) {
        f16x8 pk;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float x0 = sacc[ks >> 1][8 * (ks & 1) + e];
          const float x1 = sacc[ks >> 1][8 * (ks & 1) + e + 1];
          f32x2 pr = {__builtin_amdgcn_exp2f(__builtin_fmaf(x0, c2, -base)),
                      __builtin_amdgcn_exp2f(__builtin_fmaf(x1, c2, -base))};
          f16x2 pair = __builtin_convertvector(pr, f16x2);
          pk[e] = pair[0];
          pk[e + 1] = pair[1];
          l_i += (float)pair[0] + (float)pair[1];
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const char* vp = vptr + ks * 16 * VROWB + db * 64;
          s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(vp));
          s16x4 a2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(vp + 8 * VROWB));
          f16x4 h1 = __builtin_bit_cast(f16x4, a1), h2 = __builtin_bit_cast(f16x4, a2);
          f16x8 a = {h1[0], h1[1], h1[2], h1[3], h2[0], h2[1], h2[2], h2[3]};
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pk, oacc[db], 0, 0, 0);
        }
      }
    };

    if (active && kt0 < khi && kt0 + BN > klo) {
      const bool need_mask =
          (kt0 + BN > T) || (p.causal && kt0 + BN - 1 > r0) ||
          (p.window >= 0 && (rlast - kt0 > p.window || kt0 + BN - 1 - r0 > p.window));
      if (need_mask) tile(std::true_type{});
      else tile(std::false_type{});
    }

    if (more) store_v(buf ^ 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

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

template <int D, int BN>
constexpr int fast_lds() { return 2 * (BN * D * 2 + BN * vrow_bytes<D>()); }

bool bf16_fast_kernel(int d, AttnKernelFn* fn, int* bn, int* nw, int* lds) {
  switch (d) {
    case 64: *fn = attn_bf16_kernel<64, 64, 4>; *bn = 64; *nw = 4; *lds = fast_lds<64, 64>(); return true;
    case 256: *fn = attn_bf16_kernel<256, 64, 4>; *bn = 64; *nw = 4; *lds = fast_lds<256, 64>(); return true;
    default: return false;
  }
}

}  // namespace inl
