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
//     and stored row-major; the PV product reads them transposed with
//     `ds_read_b64_tr_b16` (within 16 lanes, lane j receives element j % 4 of
//     the 8 bytes addressed by lanes 4e + j / 4, e = 0..3), so no transpose
//     is done by ALU instructions.
//   - Buffer resources bound every text's rows: loads past the text return
//     zero, so no load needs a branch.
// The kernel requires head_dim == D (64, 128 or 256); other head dims take
// the generic kernel.

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

// Byte offset in a V (fp16, row-major, D columns) tile: 16-byte chunk c of
// row r is XOR-ed with 2 * (r & 3), so the four rows one 16-lane group of a
// transposed read touches fall on four distinct 32-byte bank ranges.
template <int D>
__device__ __forceinline__ int vswz(int r, int c) {
  return r * (D * 2) + ((c ^ ((r & 3) << 1)) << 4);
}

// D = 256 keeps 128 KB of LDS per workgroup (one per CU), so it is built
// for one wave per SIMD and the whole register file.
template <int D, int BN, int NW>
__global__ __launch_bounds__(NW * 64, D >= 256 ? 1 : 2) void attn_bf16_kernel(AttnParams p) {
  constexpr int NT = NW * 64;
  constexpr int CH = D / 8;               // 16-byte chunks per row
  constexpr int ROW = D * 2;              // bytes per K or V row in LDS
  constexpr int TILE = BN * ROW;          // bytes of one K (or V) tile
  constexpr int STAGE = 2 * TILE;         // K tile + V tile
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
  const int wave = tid >> 6;
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
      *reinterpret_cast<u32x4*>(sV + vswz<D>(row, c)) = o;
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

  for (int t = lo_t; t < hi_t; ++t) {
    const int buf = (t - lo_t) & 1;
    const bool more = t + 1 < hi_t;
    if (more) issue(t + 1, buf ^ 1);

    const int kt0 = t * BN;
    if (active && kt0 < khi && kt0 + BN > klo) {
      const char* sK = smem + buf * STAGE;
      const char* sV = sK + TILE;

      f32x16 sacc[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
        const int krow = kb * 32 + lq;
#pragma unroll
        for (int st = 0; st < D / 16; ++st) {
          bf16x8 a = *reinterpret_cast<const bf16x8*>(sK + krow * ROW + (((2 * st + hf) ^ (krow & 7)) << 4));
          sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, __builtin_bit_cast(bf16x8, qreg[st]), sacc[kb], 0, 0, 0);
        }
      }

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

      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
      mx = fmaxf(mx, wave_xor32(mx));
      const float m_new = fmaxf(m_i, mx * c2);
      const float base = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_i - base);
      m_i = m_new;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
        l_i *= alpha;
#pragma unroll
        for (int i = 0; i < NDB; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[i][r] *= alpha;
      }

      f16x8 pk[BN / 16];
      const f16x2 ones = {(f16)1.0f, (f16)1.0f};
#pragma unroll
      for (int ks = 0; ks < BN / 16; ++ks) {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const float x0 = sacc[ks >> 1][8 * (ks & 1) + e];
          const float x1 = sacc[ks >> 1][8 * (ks & 1) + e + 1];
          f32x2 pr = {__builtin_amdgcn_exp2f(__builtin_fmaf(x0, c2, -base)),
                      __builtin_amdgcn_exp2f(__builtin_fmaf(x1, c2, -base))};
          f16x2 pair = __builtin_convertvector(pr, f16x2);
          pk[ks][e] = pair[0];
          pk[ks][e + 1] = pair[1];
          l_i = __builtin_amdgcn_fdot2(pair, ones, l_i, false);
        }
      }

      // O^T += V^T . P^T; A operand = two transposed 4-key reads per lane.
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        const int col = db * 32 + 16 * (g16 & 1) + 4 * (j16 & 3);
#pragma unroll
        for (int ks = 0; ks < BN / 16; ++ks) {
          const int row1 = ks * 16 + 4 * hf + (j16 >> 2);
          const int row2 = row1 + 8;
          const int off1 = vswz<D>(row1, col >> 3) + (col & 7) * 2;
          const int off2 = vswz<D>(row2, col >> 3) + (col & 7) * 2;
          s16x4 a1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(sV + off1));
          s16x4 a2 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) s16x4*)(sV + off2));
          f16x4 h1 = __builtin_bit_cast(f16x4, a1), h2 = __builtin_bit_cast(f16x4, a2);
          f16x8 a = {h1[0], h1[1], h1[2], h1[3], h2[0], h2[1], h2[2], h2[3]};
          oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pk[ks], oacc[db], 0, 0, 0);
        }
      }
    }

    if (more) store_v(buf ^ 1);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }

  if (!active || qrow >= T) return;
  const float l_tot = l_i + wave_xor32(l_i);
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

bool bf16_fast_kernel(int d, AttnKernelFn* fn, int* bn, int* nw, int* lds) {
  switch (d) {
    case 64: *fn = attn_bf16_kernel<64, 64, 4>; *bn = 64; *nw = 4; *lds = 2 * 2 * 64 * 64 * 2; return true;
    case 128: *fn = attn_bf16_kernel<128, 64, 4>; *bn = 64; *nw = 4; *lds = 2 * 2 * 64 * 128 * 2; return true;
    case 256: *fn = attn_bf16_kernel<256, 64, 4>; *bn = 64; *nw = 4; *lds = 2 * 2 * 64 * 256 * 2; return true;
    default: return false;
  }
}

}  // namespace inl
