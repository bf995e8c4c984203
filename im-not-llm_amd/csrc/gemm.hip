// Plain bf16 GEMM on the matrix cores (gfx950): the encoder's projections
//
//   y[m, n] = alpha * sum_k x[m, k] * w[n, k]  (+ beta * y[m, n])
//
// in the row-major, bias-free Linear convention of the reference
// (candle_nn::Linear via linear_no_bias, crates/inl-text/src/qwen3/mod.rs:99-104,
// crates/inl-text/src/gemma2.rs:233-283): x [M, K] rows, w [N, K] rows (the
// checkpoint's [out, in] layout), y [M, N] rows in f32 or bf16, f32
// accumulation. No workspace, no allocation, no per-shape tuning, nothing
// synchronised: a call is one kernel launch, so the same call works under
// graph capture and for every token count M.
//
// Kernel: 256 x 256 output tiles, 8 waves (two per SIMD) as 2 (w rows, i.e.
// output columns) x 4 (x rows), each wave 128 x 64 = 4 x 2 blocks of
// v_mfma_f32_32x32x16_bf16 (the w block is the MFMA's row operand, the x
// block its column operand, so a lane's accumulator holds one output row and
// four runs of four consecutive output columns). The K
// loop runs through a 3-stage LDS ring of 32-wide k slices (32 KiB a stage),
// filled by direct global -> LDS loads three stages ahead; each stage's MFMA
// operands are read into registers one stage ahead. The workgroup is
// persistent: its tiles form one stream of stages, so the next tile's first
// loads are in flight while the current tile's epilogue stores run. The
// epilogue goes through 4 KiB of LDS per wave, 32 rows x 128 bytes at a
// time, so that every store instruction writes eight whole 128-byte row
// segments (stores straight from the accumulator layout write 32-byte pieces
// of 32 rows and took a third of the kernel's time).
//
// Gated epilogues (the GEGLU gates of EmbeddingGemma 2, gemma2.rs:249-254 and
// :279-283, fused so that the gate and up products never reach memory):
//   - GEGLU: w holds gate rows [0, n) then up rows [n, 2n) (the stacked
//     gate/up projection); y[m, c] = gelu_tanh(x . gate_c) * (x . up_c). A
//     tile covers 128 output columns and reads 128 gate and 128 up rows,
//     ordered in its LDS as alternating 16-row chunks, so each 32-row MFMA
//     block is 16 gate rows then the 16 matching up rows and a lane holds
//     both factors of its outputs;
//   - GELU x multiplier: y[m, c] = gelu_tanh(x . w_c) * mul[m, c].
// gelu_tanh(v) = v / 2 * (1 + tanh(sqrt(2 / pi) * (v + 0.044715 v^3))) in f32.
//
// Tile order: workgroup b runs on XCD b % 8. The tiles, m-tile major (all
// n-tiles of one 256-row block of x in a row), are cut into 8 contiguous
// ranges, one per XCD, and each XCD's workgroups take every 32nd tile of its
// range: the ~32 tiles an XCD runs at one time share their x rows (read from
// HBM once, then from that XCD's 4 MB L2), and w (at most a few MB) stays in
// L2 across the range.
#include <algorithm>
#include <type_traits>

#include "../../include/inl_encoder.h"
#include "attn_stream.hpp"

namespace inl {

namespace {

constexpr int GM_BN = 256;    // w rows (output columns) per tile: 2 waves x 128
constexpr int GM_BK = 32;     // k per LDS stage (64-byte rows)
constexpr int GM_ROW = GM_BK * 2;
constexpr int GM_W = GM_BN * GM_ROW;            // 16 KiB of w rows per stage
constexpr int GM_STG = 4096;                    // per-wave epilogue staging: 32 rows x 128 bytes
constexpr int GM_XCDS = 8;

// Kernel shape: NW waves as 2 (w rows) x NW / 2 (x rows), each 128 x 64;
// an LDS ring of STAGES k slices; WPC workgroups per CU.
template <int NW_, int STAGES_, int WPC_>
struct GemmShape {
  static constexpr int NW = NW_;
  static constexpr int WMW = NW / 2;                // waves along x
  static constexpr int BM = WMW * 64;               // x rows (output rows) per tile
  static constexpr int STAGES = STAGES_;
  static constexpr int WPC = WPC_;
  static constexpr int X = BM * GM_ROW;
  static constexpr int STAGE = GM_W + X;
  static constexpr int BLOCKS = STAGE / 1024;       // 1 KiB direct-load blocks per stage
  static constexpr int PER_WAVE = BLOCKS / NW;
  static constexpr int W_PER_WAVE = GM_W / 1024 / NW;
  static constexpr int RING = STAGES * STAGE;
  static constexpr int LDS = RING + NW * GM_STG;
  static_assert(BLOCKS % NW == 0 && (GM_W / 1024) % NW == 0, "the direct loads split evenly over the waves");
  static_assert(NW % 2 == 0, "w blocks of one wave share its parity (GEGLU)");
  static_assert(STAGES >= 2 && (STAGES - 1) * PER_WAVE <= 63, "vmcnt range");
};
// Shape 0: 8 waves, 256 x 256 tiles, 3 stages, one workgroup per CU (128 KiB
// LDS). Shape 1: 4 waves, 128 x 256 tiles, 2 stages, two workgroups per CU
// (64 KiB each), so that one workgroup computes while the other drains its
// tile's stores. Outputs of at most 256 columns (one n-tile per 256 rows of
// x, whose rows then stream from HBM with no reuse) run on shape 1: at
// 139,124 rows 7-8 % faster than shape 0, whose 544 tiles make 2.1 rounds
// over 256 CUs; wider outputs run on shape 0 (shape 1 was 4-15 % slower).
template <int SH>
using GemmShapeOf = std::conditional_t<SH == 1, GemmShape<4, 2, 2>, GemmShape<8, 3, 1>>;

enum GemmEpi { EPI_PLAIN = 0, EPI_GEGLU = 1, EPI_GELU_MUL = 2 };

struct GemmParams {
  const char* x;
  const char* w;
  char* y;
  const char* mul;          // EPI_GELU_MUL: bf16 [m, n] rows of ms elements
  int64_t ms;
  int64_t m;
  int32_t n, k;
  int64_t xs_b, ws_b, ys;   // x and w row strides in bytes, y row stride in elements
  float alpha, beta;
  int32_t n_tiles_n;        // tiles along n
  int64_t n_tiles;          // all tiles
  int64_t per_xcd;          // tiles per XCD range (the last ranges may be short)
  int32_t wg_per_xcd;       // workgroups per XCD
};

// 16-byte chunk c (of 4) of tile row r sits at r * 64 + ((c ^ ((r >> 2) & 3)) << 4):
// the 16 rows one ds_read_b128 pass touches then cover all 64 banks.
__device__ __forceinline__ uint32_t gm_swz(int r, int c) { return r * GM_ROW + ((c ^ ((r >> 2) & 3)) << 4); }

__device__ __forceinline__ float gelu_tanh(float v) {
  return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
}

template <int SH, int EPI, bool OUT_BF16, bool ACC>
__global__ __launch_bounds__(GemmShapeOf<SH>::NW * 64, GemmShapeOf<SH>::WPC) void gemm_bf16_kernel(GemmParams p) {
  using C = GemmShapeOf<SH>;
  constexpr int GM_NW = C::NW, GM_BM = C::BM, GM_STAGES = C::STAGES, GM_STAGE = C::STAGE;
  constexpr int GM_PER_WAVE = C::PER_WAVE, GM_RING = C::RING;
  // output columns per tile: a GEGLU tile's 256 w rows are 128 gate + 128 up
  constexpr int BNO = EPI == EPI_GEGLU ? GM_BN / 2 : GM_BN;
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int xcd = blockIdx.x % GM_XCDS;
  const int slot = blockIdx.x / GM_XCDS;
  const int64_t first = (int64_t)xcd * p.per_xcd;
  const int64_t last = min(first + p.per_xcd, p.n_tiles);   // this XCD's range [first, last)
  const int64_t t0 = first + slot;
  if (t0 >= last) return;
  const int my_tiles = (int)((last - 1 - t0) / p.wg_per_xcd + 1);
  const int kst = p.k / GM_BK;
  const int total = my_tiles * kst;

  const uint32_t lds0 = lds_addr(smem);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave / C::WMW, wm = wave % C::WMW;
  const int l32 = lane & 31, hf = lane >> 5;

  // per-lane offsets of this wave's direct-load blocks inside a tile: blocks
  // {wave, wave + NW, ...} of the stage, w rows (blocks 0-15) then x rows
  uint32_t goff[GM_PER_WAVE];
#pragma unroll
  for (int i = 0; i < GM_PER_WAVE; ++i) {
    const int blk = wave + GM_NW * i;
    const int r = lane >> 2, cp = lane & 3;
    const int c = cp ^ ((r >> 2) & 3);
    const bool is_w = i < C::W_PER_WAVE;
    // GEGLU: w block blk is 16-row chunk blk / 2 of the gate rows (blk even)
    // or of the up rows (blk odd); every w block of a wave has the wave's parity
    const int row = (is_w ? (EPI == EPI_GEGLU ? blk >> 1 : blk) : blk - GM_W / 1024) * 16 + r;
    goff[i] = (uint32_t)row * (uint32_t)(is_w ? p.ws_b : p.xs_b) + c * 16;
  }
  // The descriptors of a tile start at its first x row / w row, so no offset
  // exceeds 32 bits whatever M is; rows past M or N read as zero.
  auto tile_of = [&](int j, int64_t* mt, int* nt) __attribute__((always_inline)) {
    const int64_t t = t0 + (int64_t)j * p.wg_per_xcd;
    *mt = t / p.n_tiles_n;
    *nt = (int)(t - *mt * p.n_tiles_n);
  };
  auto rsrc_x = [&](int j) __attribute__((always_inline)) {
    int64_t mt;
    int nt;
    tile_of(j, &mt, &nt);
    const int64_t r0 = mt * GM_BM;
    const int64_t rows = min((int64_t)GM_BM, p.m - r0);
    return pp_rsrc_words(p.x + r0 * p.xs_b, (uint32_t)(rows * p.xs_b));
  };
  // this wave's w descriptor: the tile's w rows, or (GEGLU) its gate rows
  // (even waves) or up rows (odd waves)
  auto rsrc_w = [&](int j) __attribute__((always_inline)) {
    int64_t mt;
    int nt;
    tile_of(j, &mt, &nt);
    const int r0 = nt * BNO;
    const int rows = min(BNO, p.n - r0);
    const int64_t first = EPI == EPI_GEGLU && (wave & 1) ? (int64_t)p.n + r0 : (int64_t)r0;
    return pp_rsrc_words(p.w + first * p.ws_b, (uint32_t)((int64_t)rows * p.ws_b));
  };
  const i32x4 none = pp_rsrc_words(p.x, 0);   // loads past the last stage read zeros

  // The load cursor (tile ld_j, k stage ld_ks) runs up to three stages ahead
  // of the MFMA cursor, possibly into the next tile; it carries that tile's
  // descriptors.
  int ld_j = 0, ld_ks = 0, ld_slot = 0;
  i32x4 xrs = rsrc_x(0), wrs = rsrc_w(0);
  auto issue = [&]() __attribute__((always_inline)) {
    const uint32_t st = lds0 + (uint32_t)ld_slot * GM_STAGE;
    const bool live = ld_j < my_tiles;
    const uint32_t koff = (uint32_t)ld_ks * GM_ROW;
#pragma unroll
    for (int i = 0; i < GM_PER_WAVE; ++i) {
      const int blk = wave + GM_NW * i;
      const bool is_w = i < C::W_PER_WAVE;
      dma_b128(live ? (is_w ? wrs : xrs) : none, st + blk * 1024, goff[i] + koff);
    }
    if (++ld_slot == GM_STAGES) ld_slot = 0;
    if (++ld_ks == kst) {
      ld_ks = 0;
      if (++ld_j < my_tiles) {
        xrs = rsrc_x(ld_j);
        wrs = rsrc_w(ld_j);
      }
    }
  };

  // fragment addresses (stage 0): w rows wn*128 + a*32 + l32, x rows wm*64 + b*32 + l32
  uint32_t fa[4][2], fb[2][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int a = 0; a < 4; ++a) fa[a][ks] = opaque(lds0 + gm_swz(wn * 128 + a * 32 + l32, 2 * ks + hf));
#pragma unroll
    for (int b = 0; b < 2; ++b) fb[b][ks] = opaque(lds0 + GM_W + gm_swz(wm * 64 + b * 32 + l32, 2 * ks + hf));
  }

  f32x16 acc[4][2];
  const f32x16 zero = {};
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[a][b] = zero;

  // MFMA operands of one 16-wide k step: 4 w blocks and 2 x blocks
  struct Half {
    u32x4 a[4], b[2];
  };
  int rd_slot = 0;   // LDS slot of the stage whose fragments are read next
  auto read_half = [&](int ks, Half& f) __attribute__((always_inline)) {
    const uint32_t so = (uint32_t)rd_slot * GM_STAGE;
#pragma unroll
    for (int a = 0; a < 4; ++a) f.a[a] = lds_load<u32x4>(fa[a][ks] + so);
#pragma unroll
    for (int b = 0; b < 2; ++b) f.b[b] = lds_load<u32x4>(fb[b][ks] + so);
  };
  auto mfmas = [&](const Half& f) __attribute__((always_inline)) {
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b)
        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, f.a[a]),
                                                            __builtin_bit_cast(bf16x8, f.b[b]), acc[a][b], 0, 0, 0);
  };
  int mm_j = 0, mm_ks = 0;   // the MFMA cursor
  // Epilogue staging: this wave's 32 rows x 128 bytes; 16-byte chunk c of
  // row r at r * 128 + ((c ^ ((r >> 1) & 7)) << 4), so that 16 lanes writing
  // one chunk of 16 rows, and 16 lanes reading 8 chunks of 2 rows, each touch
  // all 64 banks once.
  const uint32_t stg = lds0 + GM_RING + (uint32_t)wave * GM_STG;
  auto stg_at = [&](int r, int c) __attribute__((always_inline)) {
    return stg + (uint32_t)r * 128 + (((uint32_t)c ^ (((uint32_t)r >> 1) & 7)) << 4);
  };
  // The staging holds bf16 outputs (64 columns) when they are final, and f32
  // (32 columns) otherwise: f32 outputs, and bf16 outputs that still add
  // beta * y (rounded once, after the addition).
  constexpr bool STG16 = OUT_BF16 && !ACC;
  constexpr int STG_COLS = STG16 ? 64 : 32;
  // Rows row0 .. row0 + 31 of the staged block, STG_COLS columns from output
  // column col0, to global memory: lane L stores chunk L % 8 of rows L / 8 +
  // 8 j. Rows past m and chunks past n are dropped.
  auto flush = [&](int64_t row0, int col0) __attribute__((always_inline)) {
    constexpr int EPC = STG16 ? 8 : 4;   // elements per 16-byte staged chunk
    const int c = lane & 7;
    const int col = col0 + c * EPC;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = (lane >> 3) + 8 * j;
      const u32x4 v = lds_load<u32x4>(stg_at(r, c));
      const int64_t row = row0 + r;
      if (row < p.m && col < p.n) {
        char* dst = p.y + (row * p.ys + col) * (OUT_BF16 ? 2 : 4);
        if constexpr (STG16) {
          *reinterpret_cast<u32x4*>(dst) = v;
        } else {
          f32x4 t = __builtin_bit_cast(f32x4, v);
          if constexpr (OUT_BF16) {   // ACC: add beta * y, then round
            const bf16x4 o = *reinterpret_cast<const bf16x4*>(dst);
            bf16x4 r4;
#pragma unroll
            for (int e = 0; e < 4; ++e) r4[e] = (bf16)(t[e] + p.beta * (float)o[e]);
            *reinterpret_cast<bf16x4*>(dst) = r4;
          } else {
            if constexpr (ACC) {
              const f32x4 o = *reinterpret_cast<const f32x4*>(dst);
#pragma unroll
              for (int e = 0; e < 4; ++e) t[e] += p.beta * o[e];
            }
            *reinterpret_cast<f32x4*>(dst) = t;
          }
        }
      }
    }
  };
  // 4 output values of this lane's row at staged column chunk_col (a multiple of 4)
  auto put4 = [&](int chunk_col, f32x4 v) __attribute__((always_inline)) {
    if constexpr (STG16) {
      const f32x2 lo = {v[0], v[1]}, hi = {v[2], v[3]};
      const u32x2 w = {__builtin_bit_cast(uint32_t, __builtin_convertvector(lo, bf16x2)),
                       __builtin_bit_cast(uint32_t, __builtin_convertvector(hi, bf16x2))};
      lds_store<u32x2>(stg_at(l32, chunk_col >> 3) + ((chunk_col & 7) << 1), w);
    } else {
      // (whole-vector casts: hipcc miscompiles __builtin_bit_cast of a vector
      // element lvalue such as v[e], broadcasting one element)
      lds_store<u32x4>(stg_at(l32, chunk_col >> 2), __builtin_bit_cast(u32x4, v));
    }
  };
  // tile done: acc[a][b][4 * g + e] is product (row wm*64 + b*32 + l32,
  // w row wn*128 + a*32 + 8*g + 4*hf + e) of the tile
  auto tile_end = [&]() __attribute__((always_inline)) {
    if (++mm_ks != kst) return;
    mm_ks = 0;
    int64_t mt;
    int nt;
    tile_of(mm_j++, &mt, &nt);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int64_t row0 = mt * GM_BM + wm * 64 + b * 32;
      if constexpr (EPI == EPI_GEGLU) {
        // block wn*4 + a: gate rows 0-15 and their up rows 16-31 give output
        // columns 16 (wn*4 + a) + 0..15 of the tile: all four blocks are 64
        // bf16 or f32 columns, staged 128 bytes (32 f32 columns) at a time
        constexpr int PER = STG_COLS / 16;   // a-blocks (16 outputs each) per staging
#pragma unroll
        for (int a0 = 0; a0 < 4; a0 += PER) {
#pragma unroll
          for (int a = a0; a < a0 + PER; ++a)
#pragma unroll
            for (int g = 0; g < 2; ++g) {
              f32x4 v;
#pragma unroll
              for (int e = 0; e < 4; ++e)
                v[e] = gelu_tanh(p.alpha * acc[a][b][4 * g + e]) * (p.alpha * acc[a][b][4 * (g + 2) + e]);
              put4((a - a0) * 16 + 8 * g + 4 * hf, v);
            }
          flush(row0, nt * BNO + wn * 64 + a0 * 16);
        }
      } else {
        constexpr int PER = STG_COLS / 32;   // a-blocks (32 columns each) per staging
#pragma unroll
        for (int a0 = 0; a0 < 4; a0 += PER) {
#pragma unroll
          for (int a = a0; a < a0 + PER; ++a)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              f32x4 v;
              if constexpr (EPI == EPI_GELU_MUL) {
                const int64_t row = row0 + l32;
                const int col = nt * BNO + wn * 128 + a * 32 + 8 * g + 4 * hf;
                bf16x4 mv = {};
                if (row < p.m && col < p.n) mv = *reinterpret_cast<const bf16x4*>(p.mul + (row * p.ms + col) * 2);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = gelu_tanh(p.alpha * acc[a][b][4 * g + e]) * (float)mv[e];
              } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = p.alpha * acc[a][b][4 * g + e];
              }
              put4((a - a0) * 32 + 8 * g + 4 * hf, v);
            }
          flush(row0, nt * BNO + wn * 128 + a0 * 32);
        }
      }
    }
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 2; ++b) acc[a][b] = zero;
  };
  // One iteration per stage s, with h0 holding its first k step's operands:
  // read its second k step's operands while the first step's MFMAs run;
  // then wait for stage s + 1 (vmcnt) and for every wave to have read all of
  // stage s (barrier), refill stage s's LDS slot with stage s + GM_STAGES, and read
  // stage s + 1's first k step while the second step's MFMAs run.
  Half h0, h1;
  auto step = [&]() __attribute__((always_inline)) {
    read_half(1, h1);
    mfmas(h0);
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"((GM_STAGES - 2) * GM_PER_WAVE) : "memory");
    lds_barrier();
    issue();
    if (++rd_slot == GM_STAGES) rd_slot = 0;
    read_half(0, h0);
    mfmas(h1);
    tile_end();
  };

#pragma unroll
  for (int i = 0; i < GM_STAGES; ++i) issue();
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"((GM_STAGES - 1) * GM_PER_WAVE) : "memory");   // stage 0
  lds_barrier();
  read_half(0, h0);
  for (int st = 0; st < total; ++st) step();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the dummy loads past the end
}

template <int SH, int E, bool B, bool A>
const void* gemm_fn() {
  return (const void*)gemm_bf16_kernel<SH, E, B, A>;
}

// The shape-dependent part of a launch: tile counts, workgroups and kernel.
template <int SH>
int gemm_launch_shape(GemmParams p, int epi, bool bf, bool acc, int64_t m, int64_t k, int cus, void* stream) {
  using C = GemmShapeOf<SH>;
  p.n_tiles = ((m + C::BM - 1) / C::BM) * p.n_tiles_n;
  p.per_xcd = (p.n_tiles + GM_XCDS - 1) / GM_XCDS;
  // C::WPC workgroups per CU, at most one per tile of an XCD's range
  const int64_t per_xcd_wg = std::max<int64_t>(1, std::min<int64_t>(cus / GM_XCDS * C::WPC, p.per_xcd));
  p.wg_per_xcd = (int32_t)per_xcd_wg;
  if ((int64_t)(p.per_xcd + per_xcd_wg - 1) / per_xcd_wg * (k / GM_BK) >= ((int64_t)1 << 31))
    return fail(INL_E_UNSUPPORTED, "gemm: too many k stages per workgroup");
  const void* fn = nullptr;
  switch (epi * 4 + (bf ? 2 : 0) + (acc ? 1 : 0)) {
#define INL_GEMM_CASE(E, B, A) \
  case E * 4 + (B ? 2 : 0) + (A ? 1 : 0): fn = gemm_fn<SH, E, B, A>(); break;
    INL_GEMM_CASE(EPI_PLAIN, false, false)
    INL_GEMM_CASE(EPI_PLAIN, false, true)
    INL_GEMM_CASE(EPI_PLAIN, true, false)
    INL_GEMM_CASE(EPI_PLAIN, true, true)
    INL_GEMM_CASE(EPI_GEGLU, false, false)
    INL_GEMM_CASE(EPI_GEGLU, true, false)
    INL_GEMM_CASE(EPI_GELU_MUL, false, false)
    INL_GEMM_CASE(EPI_GELU_MUL, true, false)
#undef INL_GEMM_CASE
    default:
      return fail(INL_E_UNSUPPORTED, "gemm: the gated epilogues take beta = 0");
  }
  int rc = set_max_dynamic_lds(fn, C::LDS);
  if (rc) return rc;
  void* args[] = {&p};
  INL_HIP_TRY(hipLaunchKernel(fn, dim3((unsigned)(per_xcd_wg * GM_XCDS)), dim3(C::NW * 64), args, C::LDS,
                              (hipStream_t)stream));
  return INL_OK;
}

// Launch for every epilogue; `n` is the output width (GEGLU: w has 2n rows).
int gemm_launch(int epi, int64_t m, int64_t n, int64_t k, const void* x, int64_t x_stride, const void* w,
                int64_t w_stride, const void* mul, int64_t mul_stride, int32_t out_dtype, void* y, int64_t y_stride,
                float alpha, float beta, void* stream) {
  if (m < 0 || n <= 0 || k <= 0) return fail(INL_E_INVALID, "gemm: m must be >= 0, n and k > 0");
  if (!dtype_ok(out_dtype)) return fail(INL_E_INVALID, "gemm: out_dtype must be f32 or bf16");
  if (k % GM_BK || n % 8)
    return fail(INL_E_UNSUPPORTED, "gemm: k must be a multiple of 32 and n a multiple of 8");
  if (n > (1 << 29) || k > (1 << 20)) return fail(INL_E_UNSUPPORTED, "gemm: n or k too large");
  const int64_t xs = x_stride ? x_stride : k, ws = w_stride ? w_stride : k, ys = y_stride ? y_stride : n;
  const int64_t ms = mul_stride ? mul_stride : n;
  if (xs < k || ws < k || ys < n || (epi == EPI_GELU_MUL && ms < n))
    return fail(INL_E_INVALID, "gemm: a row stride is shorter than its row");
  if (xs % 8 || ws % 8 || ys % 8 || (epi == EPI_GELU_MUL && ms % 4))
    return fail(INL_E_UNSUPPORTED, "gemm: row strides must be multiples of 8 elements (the multiplier's of 4)");
  if (m == 0) return INL_OK;
  if (!x || !w || !y || (epi == EPI_GELU_MUL && !mul)) return fail(INL_E_INVALID, "gemm: NULL x, w, y or multiplier");
  if (((uintptr_t)x & 15) || ((uintptr_t)w & 15) || ((uintptr_t)y & 15) || ((uintptr_t)mul & 7))
    return fail(INL_E_INVALID, "gemm: x, w and y must be 16-byte aligned, the multiplier 8-byte aligned");
  // each tile's descriptor spans at most 256 rows of x or w
  if ((int64_t)256 * xs * 2 >= ((int64_t)1 << 32) || (int64_t)GM_BN * ws * 2 >= ((int64_t)1 << 32))
    return fail(INL_E_UNSUPPORTED, "gemm: row strides too large for a tile's 32-bit buffer range");
  int dev = 0, cus = 0;
  INL_HIP_TRY(hipGetDevice(&dev));
  INL_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int bno = epi == EPI_GEGLU ? GM_BN / 2 : GM_BN;
  GemmParams p{};
  p.x = (const char*)x;
  p.w = (const char*)w;
  p.y = (char*)y;
  p.mul = (const char*)mul;
  p.ms = ms;
  p.m = m;
  p.n = (int32_t)n;
  p.k = (int32_t)k;
  p.xs_b = xs * 2;
  p.ws_b = ws * 2;
  p.ys = ys;
  p.alpha = alpha;
  p.beta = beta;
  p.n_tiles_n = (int32_t)((n + bno - 1) / bno);
  const bool bf = out_dtype == INL_BF16, acc = beta != 0.f;
  if (p.n_tiles_n == 1) return gemm_launch_shape<1>(p, epi, bf, acc, m, k, cus, stream);
  return gemm_launch_shape<0>(p, epi, bf, acc, m, k, cus, stream);
}

}  // namespace

}  // namespace inl

extern "C" int inl_gemm_bf16_fwd(int64_t m, int64_t n, int64_t k, const void* x, int64_t x_stride, const void* w,
                                 int64_t w_stride, int32_t out_dtype, void* y, int64_t y_stride, float alpha,
                                 float beta, void* stream) {
  return inl::gemm_launch(inl::EPI_PLAIN, m, n, k, x, x_stride, w, w_stride, nullptr, 0, out_dtype, y, y_stride,
                          alpha, beta, stream);
}

extern "C" int inl_gemm_bf16_gated_fwd(int64_t m, int64_t n, int64_t k, const void* x, int64_t x_stride,
                                       const void* w, int64_t w_stride, int32_t mode, const void* mul,
                                       int64_t mul_stride, int32_t out_dtype, void* y, int64_t y_stride,
                                       void* stream) {
  using namespace inl;
  if (mode != INL_GATE_GEGLU && mode != INL_GATE_GELU_MUL)
    return fail(INL_E_INVALID, "gemm: mode must be INL_GATE_GEGLU or INL_GATE_GELU_MUL");
  return gemm_launch(mode == INL_GATE_GEGLU ? EPI_GEGLU : EPI_GELU_MUL, m, n, k, x, x_stride, w, w_stride, mul,
                     mul_stride, out_dtype, y, y_stride, 1.f, 0.f, stream);
}
