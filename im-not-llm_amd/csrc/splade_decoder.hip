// Fused SPLADE decoder GEMM + per-text max (gfx950, bf16 MFMA).
//
// The SPLADE epilogue of the sparse engine (crates/inl-sparse/src/
// modernbert.rs:657-662 `project`, :806-872 `pool_states`) multiplies every
// speaking position's MLM-head output [S, H] by the bias-free decoder weight
// [V, H]^T and keeps, per text and term, only the maximum over the text's
// positions (bias, shift, relu and log are monotone, so they run once per
// text afterwards). At the benchmark's config 4 that is a 135,764 x 50,002 x
// 768 product (10.4 TFLOP) whose f32 logits would be 27 GB; here they never
// leave the registers:
//
//   out[r, v] = max over p in [offs[r], offs[r+1]) of  head[p, :] . w[v, :]
//
// (-inf for a text without speaking positions, as the reference's `silent`
// row). One workgroup owns one (text, 512-term tile) and walks the text's
// positions in chunks of 128: for each chunk it runs the K = H loop through
// LDS (32-wide k slices, 3 stages, direct global -> LDS loads three stages
// ahead, each stage's MFMA operands read into registers one stage ahead) and
// folds the chunk's 128 x 512 product into a running column maximum held in
// registers. 8 waves as 2 (positions) x 4 (terms),
// each 64 x 128 = 2 x 4 MFMA blocks of 32 x 32 (v_mfma_f32_32x32x16_bf16,
// f32 accumulation): a lane holds one term column and 16 position rows of a
// block, so the max over positions is lane-local plus one exchange between
// the lane halves. The workgroups one XCD runs at a time share a term tile,
// whose decoder rows then stay in that XCD's L2 (see splade_units).
#include <algorithm>
#include <numeric>
#include <queue>
#include <vector>

#include "../../include/inl_encoder.h"
#include "attn_stream.hpp"

namespace inl {

namespace {

constexpr int SD_BM = 128;   // positions per chunk
constexpr int SD_BN = 512;   // vocabulary terms per workgroup
constexpr int SD_BK = 32;    // k per LDS stage (64-byte rows)
constexpr int SD_STAGES = 3;
constexpr int SD_ROW = SD_BK * 2;
constexpr int SD_A = SD_BM * SD_ROW;            // 8 KiB
constexpr int SD_B = SD_BN * SD_ROW;            // 32 KiB
constexpr int SD_STAGE = SD_A + SD_B;           // 40 KiB
constexpr int SD_BLOCKS = SD_STAGE / 1024;      // 1 KiB direct-load blocks per stage
constexpr int SD_NW = 8;
constexpr int SD_PER_WAVE = SD_BLOCKS / SD_NW;  // 5
constexpr int SD_LDS = SD_STAGES * SD_STAGE + 4 * 4 * 32 * 4;  // + the cross-wave max exchange

struct SpladeDecParams {
  const char* head;
  const char* w;
  float* out;
  const int2* units;      // per workgroup: {text, term tile}, XCD-ordered; text -1 = idle
  const int2* texts;      // per text: {first position, positions}
  int32_t hidden;         // K, a multiple of 32
  int32_t vocab;
  uint32_t head_bytes, w_bytes;  // descriptor ranges
  uint32_t hs_b, ws_b;           // row strides in bytes
};

static_assert(SD_BLOCKS % SD_NW == 0, "the direct loads split evenly over the waves");

// 16-byte chunk c (of 4) of tile row r sits at r * 64 + ((c ^ ((r >> 2) & 3)) << 4):
// the 16 rows one pass of a ds_read_b128 touches then cover all 64 banks.
__device__ __forceinline__ uint32_t sd_swz(int r, int c) { return r * SD_ROW + ((c ^ ((r >> 2) & 3)) << 4); }

__global__ __launch_bounds__(SD_NW * 64) void splade_decoder_max_kernel(SpladeDecParams p) {
  extern __shared__ __attribute__((aligned(1024))) char smem[];
  const int2 un = p.units[blockIdx.x];
  if (un.x < 0) return;
  const int2 tx = p.texts[un.x];
  const int seg = __builtin_amdgcn_readfirstlane(tx.x);
  const int T = __builtin_amdgcn_readfirstlane(tx.y);
  const int v0 = __builtin_amdgcn_readfirstlane(un.y) * SD_BN;
  const uint32_t lds0 = lds_addr(smem);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 2, wn = wave & 3;
  const int l32 = lane & 31, hf = lane >> 5;

  const int kst = p.hidden / SD_BK;                 // stages per chunk
  const int chunks = (T + SD_BM - 1) / SD_BM;
  const int total = chunks * kst;

  const i32x4 ars = pp_rsrc_words(p.head, p.head_bytes);
  const i32x4 brs = pp_rsrc_words(p.w, p.w_bytes);
  const i32x4 none = pp_rsrc_words(p.head, 0);      // loads past the end read zeros

  // this wave's direct-load blocks: {wave, wave + 8, ...} of the 40 per stage
  uint32_t goff[SD_PER_WAVE];
  bool is_a[SD_PER_WAVE];
#pragma unroll
  for (int i = 0; i < SD_PER_WAVE; ++i) {
    const int blk = wave + SD_NW * i;
    const int r = lane >> 2, cp = lane & 3;
    const int c = cp ^ ((r >> 2) & 3);
    is_a[i] = blk < SD_A / 1024;
    const int row = (is_a[i] ? blk : blk - SD_A / 1024) * 16 + r;
    goff[i] = is_a[i] ? (uint32_t)row * p.hs_b + c * 16 : (uint32_t)(v0 + row) * p.ws_b + c * 16;
  }
  const uint32_t seg_off = (uint32_t)seg * p.hs_b;
  auto issue = [&](int s) __attribute__((always_inline)) {
    const uint32_t st = lds0 + (uint32_t)(s % SD_STAGES) * SD_STAGE;
    const bool live = s < total;
    const int chunk = s / kst, ks = s - (s / kst) * kst;
    const uint32_t koff = (uint32_t)ks * SD_ROW;
    const uint32_t aoff = seg_off + (uint32_t)chunk * SD_BM * p.hs_b + koff;
#pragma unroll
    for (int i = 0; i < SD_PER_WAVE; ++i) {
      const int blk = wave + SD_NW * i;
      dma_b128(live ? (is_a[i] ? ars : brs) : none, st + blk * 1024, goff[i] + (is_a[i] ? aoff : koff));
    }
  };

  // fragment addresses (stage 0): A rows wm*64 + mb*32 + l32, B rows wn*128 + nb*32 + l32
  uint32_t fa[2][2], fb[4][2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) fa[mb][ks] = opaque(lds0 + sd_swz(wm * 64 + mb * 32 + l32, 2 * ks + hf));
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) fb[nb][ks] = opaque(lds0 + SD_A + sd_swz(wn * 128 + nb * 32 + l32, 2 * ks + hf));
  }

  f32x16 acc[2][4];
  const f32x16 zero = {};
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = zero;
  float rmax[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};

  // fragments of one stage: A (2 row blocks) and B (4 column blocks) for the
  // stage's two 16-wide k steps
  struct Frags {
    u32x4 a[2][2], b[4][2];
  };
  auto read_frags = [&](int st, Frags& f) __attribute__((always_inline)) {
    const uint32_t so = (uint32_t)(st % SD_STAGES) * SD_STAGE;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) f.a[mb][ks] = lds_load<u32x4>(fa[mb][ks] + so);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) f.b[nb][ks] = lds_load<u32x4>(fb[nb][ks] + so);
    }
  };
  auto mfmas = [&](const Frags& f) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, f.a[mb][ks]),
                                                                __builtin_bit_cast(bf16x8, f.b[nb][ks]),
                                                                acc[mb][nb], 0, 0, 0);
  };
  auto chunk_end = [&](int st) __attribute__((always_inline)) {
    if ((st + 1) % kst != 0) return;
    // chunk done: rows past the text's end do not count
    const int chunk = st / kst;
    const int rbase = chunk * SD_BM + wm * 64 + 4 * hf;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      float m = -INFINITY;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int row = rbase + mb * 32 + 8 * (i >> 2) + (i & 3);
          m = __builtin_elementwise_maximum(m, row < T ? acc[mb][nb][i] : -INFINITY);
        }
      rmax[nb] = __builtin_elementwise_maximum(rmax[nb], half_max(m));
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc[mb][nb] = zero;
  };
  // One iteration per stage s: stage s + 1 has landed (vmcnt) and is visible
  // (barrier), and every wave has read stage s's fragments, so its LDS slot
  // takes the loads of stage s + 3; then stage s + 1's fragments are read
  // into the spare register set while stage s's MFMAs run.
  auto step = [&](int st, const Frags& cur, Frags& nxt) __attribute__((always_inline)) {
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(SD_PER_WAVE) : "memory");
    lds_barrier();
    issue(st + 3);
    read_frags(st + 1, nxt);
    mfmas(cur);
    chunk_end(st);
  };

  issue(0);
  issue(1);
  issue(2);
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * SD_PER_WAVE) : "memory");   // stage 0
  lds_barrier();
  Frags f0, f1;
  read_frags(0, f0);
  for (int st = 0; st < total; st += 2) {
    step(st, f0, f1);
    if (st + 1 >= total) break;
    step(st + 1, f1, f0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the dummy loads past the end
  // the two position halves of each term column meet in LDS
  const uint32_t ex = lds0 + SD_STAGES * SD_STAGE + (uint32_t)(wn * 4 * 32 + l32) * 4;
  lds_barrier();
  if (wm == 1 && hf == 0)
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) lds_store<float>(ex + nb * 32 * 4, rmax[nb]);
  lds_barrier();
  if (wm == 0 && hf == 0) {
    float* o = p.out + (int64_t)un.x * p.vocab;
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int v = v0 + wn * 128 + nb * 32 + l32;
      const float m = __builtin_elementwise_maximum(rmax[nb], lds_load<float>(ex + nb * 32 * 4));
      if (v < p.vocab) o[v] = m;
    }
  }
}

// Host: the (text, term tile) units in launch order. Workgroup b runs on XCD
// b % 8, and each XCD has its own 4 MB L2. A term tile's decoder rows
// (512 x hidden, 768 KB at hidden 768) are read again for every 128-position
// chunk of every text, so the units are ordered tile-major - all texts of
// tile 0, then of tile 1, ... (texts longest first) - and dealt to the 8 XCD
// classes in contiguous runs of equal cost: the workgroups an XCD runs at
// the same time share one decoder tile in its L2, and only the head rows
// (once per tile per text) come from further out.
void splade_units(const int32_t* offs, int32_t rows, int n_tiles, std::vector<int2>* units,
                  std::vector<int2>* texts) {
  texts->resize(rows);
  std::vector<int> order(rows);
  for (int r = 0; r < rows; ++r) {
    (*texts)[r] = make_int2(offs[r], offs[r + 1] - offs[r]);
    order[r] = r;
  }
  std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return (*texts)[a].y > (*texts)[b].y; });
  auto cost = [&](int r) { return (int64_t)std::max(1, ((*texts)[r].y + SD_BM - 1) / SD_BM); };
  int64_t per_tile = 0;
  for (int r = 0; r < rows; ++r) per_tile += cost(r);
  const int64_t total = per_tile * n_tiles;
  std::vector<std::vector<int2>> cls(8);
  int64_t done = 0;
  int c = 0;
  for (int j = 0; j < n_tiles; ++j)
    for (int r : order) {
      while (c < 7 && done >= (total * (c + 1)) / 8) ++c;
      cls[c].push_back(make_int2(r, j));
      done += cost(r);
    }
  size_t longest = 0;
  for (auto& v : cls) longest = std::max(longest, v.size());
  units->assign(longest * 8, make_int2(-1, 0));
  for (int k = 0; k < 8; ++k)
    for (size_t i = 0; i < cls[k].size(); ++i) (*units)[i * 8 + k] = cls[k][i];
}

}  // namespace

}  // namespace inl

extern "C" int inl_splade_decoder_workspace_size(int32_t rows, int32_t vocab, size_t* bytes) {
  using namespace inl;
  if (!bytes || rows < 0 || vocab <= 0) return fail(INL_E_INVALID, "splade_decoder: bad arguments");
  const int64_t tiles = (vocab + SD_BN - 1) / SD_BN;
  // units: 8 classes, each spanning at most tiles / 8 + 2 tiles of `rows` units
  const int64_t units = (int64_t)rows * (tiles + 16) + 8;
  *bytes = (size_t)(units + rows) * sizeof(int2) + 256;
  return INL_OK;
}

extern "C" int inl_splade_decoder_max_fwd(int32_t rows, const int32_t* offs_host, const void* head,
                                          int64_t head_stride, int32_t hidden, const void* w_dec,
                                          int64_t w_stride, int32_t vocab, int32_t dtype, float* out,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  using namespace inl;
  if (rows < 0 || vocab <= 0 || hidden <= 0) return fail(INL_E_INVALID, "splade_decoder: bad sizes");
  if (dtype != INL_BF16) return fail(INL_E_UNSUPPORTED, "splade_decoder: the fused kernel takes bf16 head and weight");
  if (hidden % SD_BK) return fail(INL_E_UNSUPPORTED, "splade_decoder: hidden must be a multiple of 32");
  const int64_t hs = head_stride ? head_stride : hidden, wsd = w_stride ? w_stride : hidden;
  if (hs < hidden || wsd < hidden || hs % 8 || wsd % 8)
    return fail(INL_E_INVALID, "splade_decoder: row strides must cover the row in 16-byte multiples");
  if (rows == 0) return INL_OK;
  if (!offs_host || !head || !w_dec || !out || !workspace)
    return fail(INL_E_INVALID, "splade_decoder: NULL pointer");
  int64_t S = 0;
  int rc = check_cu(rows, offs_host, &S);
  if (rc) return rc;
  if ((S + SD_BM) * hs * 2 >= ((int64_t)1 << 32) || ((int64_t)vocab + SD_BN) * wsd * 2 >= ((int64_t)1 << 32))
    return fail(INL_E_UNSUPPORTED, "splade_decoder: head or weight spans 4 GiB or more");
  if (((uintptr_t)head & 15) || ((uintptr_t)w_dec & 15) || ((uintptr_t)workspace & 15))
    return fail(INL_E_INVALID, "splade_decoder: head, w_dec and workspace must be 16-byte aligned");
  const int tiles = (vocab + SD_BN - 1) / SD_BN;
  std::vector<int2> units, texts;
  splade_units(offs_host, rows, tiles, &units, &texts);
  size_t need = 0;
  rc = inl_splade_decoder_workspace_size(rows, vocab, &need);
  if (rc) return rc;
  const size_t ub = units.size() * sizeof(int2), tb = texts.size() * sizeof(int2);
  if (workspace_bytes < ub + tb || units.size() > 0x7fffffff)
    return fail(INL_E_INVALID, "splade_decoder: workspace smaller than inl_splade_decoder_workspace_size()");
  std::vector<int2> blob(units);
  blob.insert(blob.end(), texts.begin(), texts.end());
  hipStream_t st = (hipStream_t)stream;
  INL_HIP_TRY(hipMemcpyAsync(workspace, blob.data(), blob.size() * sizeof(int2), hipMemcpyHostToDevice, st));
  rc = set_max_dynamic_lds((const void*)splade_decoder_max_kernel, SD_LDS);
  if (rc) return rc;
  SpladeDecParams p{};
  p.head = (const char*)head;
  p.w = (const char*)w_dec;
  p.out = out;
  p.units = (const int2*)workspace;
  p.texts = (const int2*)workspace + units.size();
  p.hidden = hidden;
  p.vocab = vocab;
  p.head_bytes = (uint32_t)(S * hs * 2);
  p.w_bytes = (uint32_t)((int64_t)vocab * wsd * 2);
  p.hs_b = (uint32_t)(hs * 2);
  p.ws_b = (uint32_t)(wsd * 2);
  hipLaunchKernelGGL(splade_decoder_max_kernel, dim3((unsigned)units.size()), dim3(SD_NW * 64), SD_LDS, st, p);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}
