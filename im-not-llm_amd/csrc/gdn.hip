// Gated-delta-net ops of the Qwen3.5 (pplx-late) tower on gfx950: the causal
// depthwise convolution + silu, the gates, the per-token gated delta rule,
// the gated RMSNorm and the unit-lower-triangular inverse of the chunked
// rule. Reference: crates/inl-late/src/qwen3_5.rs:411-773 and the Metal
// kernels it routes to (crates/inl-late/src/late.metal, metal.rs).
//
// Rounding. The convolution, the gated norm and the inverse reproduce the
// reference kernels' operation sequence: each product, sum, cast and silu
// step rounds on its own (no contraction into fused multiply-adds, hence the
// file-wide pragma below), in the reference's order. Only transcendental
// results (exp, log) may differ from the reference's by an ulp. The rule is
// the exception: its state update uses explicit fused multiply-adds, in a
// different summation order, because it is the VALU-bound inner loop.
//
// Layout. Texts are packed (row t of the token stream belongs to the text b
// with cu[b] <= t < cu[b + 1]); each text starts from zero padding (the
// convolution) and a zero state (the rule).

#include <cmath>

#include "../../include/inl_gdn.h"
#include "attn_kernels.hpp"
#include "inl_common.hpp"
#include "lanes.hpp"

#pragma clang fp contract(off)

namespace inl {

namespace {

// Value of dtype T stored at p, widened exactly to f32.
template <typename T>
__device__ __forceinline__ float ld1(const T* p) { return (float)*p; }

// One f32 value rounded to bf16 and back with one v_cvt_pk_bf16_f32: with
// the value in the high half and +0 in the low half, the packed result is
// already the f32 bit pattern of the rounded value.
__device__ __forceinline__ float rnd1_bf16(float a) {
  return __builtin_bit_cast(float, __builtin_convertvector((f32x2){0.f, a}, bf16x2));
}

// Round an f32 to T and back (identity for f32). (rnd1_bf16 in its place
// measured 8 % slower in the gated norm, whose loads it rescheduled.)
template <typename T>
__device__ __forceinline__ float rnd(float x) { return (float)(T)x; }

// exp and division of an f32 result that is rounded to T next: exact-rounding
// library forms for f32; for bf16 the hardware forms (an ulp or two of f32
// error, which moves a bf16 rounding only when the f32 value sits within
// those ulps of a bf16 midpoint).
template <typename T>
__device__ __forceinline__ float exp_t(float x) {
  if constexpr (sizeof(T) == 2) return __expf(x);
  else return expf(x);
}
template <typename T>
__device__ __forceinline__ float div_t(float x, float d) {
  if constexpr (sizeof(T) == 2) return x * __builtin_amdgcn_rcpf(d);
  else return __fdiv_rn(x, d);
}

// Two f32 values rounded to bf16 and back with one v_cvt_pk_bf16_f32.
__device__ __forceinline__ void rnd2_bf16(float a, float b, float& ra, float& rb) {
  const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  ra = __builtin_bit_cast(float, h << 16);
  rb = __builtin_bit_cast(float, h & 0xffff0000u);
}

// candle's silu with every step rounded in T: x / (1 + exp(-x)).
template <typename T>
__device__ __forceinline__ float silu_t(float x) {
  const float e = rnd<T>(exp_t<T>(rnd<T>(-x)));
  const float d = rnd<T>(1.0f + e);
  return rnd<T>(div_t<T>(x, d));
}
// silu_t<bf16> of two values that are bf16 already (so -x needs no rounding),
// returned as the packed bf16 pair (the last rounding is the output's).
__device__ __forceinline__ uint32_t silu2_bf16(float x0, float x1) {
  const float e0 = rnd1_bf16(exp_t<bf16>(-x0)), e1 = rnd1_bf16(exp_t<bf16>(-x1));
  const float d0 = rnd1_bf16(1.0f + e0), d1 = rnd1_bf16(1.0f + e1);
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){div_t<bf16>(x0, d0), div_t<bf16>(x1, d1)},
                                                             bf16x2));
}

// Index of the text holding packed row t: the last b with cu[b] <= t
// (empty texts before it are skipped because their cu[b + 1] == cu[b] <= t).
__device__ __forceinline__ int text_of(const int32_t* cu, int n_texts, int64_t t) {
  int lo = 0, hi = n_texts;  // answer in [lo, hi)
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if ((int64_t)cu[mid] <= t) lo = mid;
    else hi = mid;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// Causal depthwise convolution + silu. A thread owns V consecutive channels
// and a run of CONV_RUN consecutive packed rows, keeping the previous
// taps - 1 input rows in registers (each input row is read once, plus a
// halo of taps - 1 rows per run). Product and sum rounded in T per tap, in
// tap order (late.metal:131-151).
// ---------------------------------------------------------------------------
constexpr int CONV_RUN = 16;
constexpr int CONV_MAX_TAPS = 8;

template <typename T, int V, int TAPS>
__global__ __launch_bounds__(256) void gdn_conv_kernel(const T* __restrict__ x, int64_t xs,
                                                       const int32_t* __restrict__ cu, int n_texts,
                                                       int64_t n_tokens, int channels,
                                                       const T* __restrict__ w, T* __restrict__ out,
                                                       int64_t os) {
  const int groups = channels / V;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int cg = (int)(gid % groups);
  const int64_t t0 = (gid / groups) * CONV_RUN;
  if (t0 >= n_tokens) return;
  const int c0 = cg * V;

  float wt[TAPS][V];
#pragma unroll
  for (int k = 0; k < TAPS; ++k)
#pragma unroll
    for (int e = 0; e < V; ++e) wt[k][e] = ld1(w + (int64_t)(c0 + e) * TAPS + k);

  // cu is clamped into [0, n_tokens]: a malformed table gives wrong rows, never an access outside x
  auto at = [&](int i) -> int64_t {
    const int64_t v = cu[i];
    return v < 0 ? 0 : (v > n_tokens ? n_tokens : v);
  };
  int b = text_of(cu, n_texts, t0);
  int64_t start = at(b), stop = at(b + 1);

  // win[j] = input row t - 1 - j (zero before the text's start); win[TAPS - 1]
  // is never read (it keeps the array non-empty for TAPS == 1)
  float win[TAPS][V];
#pragma unroll
  for (int j = 0; j < TAPS; ++j) {
    const int64_t pos = t0 - 1 - j;
    const bool in = j < TAPS - 1 && pos >= start;
    const int64_t pc = in ? pos : t0;  // a valid row: loaded unconditionally, masked after
#pragma unroll
    for (int e = 0; e < V; ++e) {
      const float v = ld1(x + pc * xs + c0 + e);
      win[j][e] = in ? v : 0.f;
    }
  }

  const int64_t t1 = t0 + CONV_RUN < n_tokens ? t0 + CONV_RUN : n_tokens;
  // Every row of the run is loaded first (rows past the end at the run's
  // last row, unused), so the loads are in flight together; the unrolled
  // loop then renames the window registers instead of moving them.
  constexpr bool VB = V == 8 && sizeof(T) == 2, VF = V == 4 && sizeof(T) == 4;
  u32x4 raw[VB ? CONV_RUN : 1];
  f32x4 rawf[VF ? CONV_RUN : 1];
#pragma unroll
  for (int i = 0; i < CONV_RUN; ++i) {
    const int64_t tc = t0 + i < t1 ? t0 + i : t1 - 1;
    if constexpr (VB) raw[i] = *reinterpret_cast<const u32x4*>(x + tc * xs + c0);
    if constexpr (VF) rawf[i] = *reinterpret_cast<const f32x4*>(x + tc * xs + c0);
  }
#pragma unroll
  for (int i = 0; i < CONV_RUN; ++i) {
    const int64_t t = t0 + i;
    if (t >= t1) break;
    if (t >= stop) {  // the next text starts here: zero padding again
      while (t >= stop && b + 1 < n_texts) { ++b; stop = at(b + 1); }
      start = t < stop ? at(b) : t;  // rows past cu[n_texts] start afresh
#pragma unroll
      for (int j = 0; j < TAPS; ++j)
#pragma unroll
        for (int e = 0; e < V; ++e) win[j][e] = 0.f;
    }
    float cur[V];
    if constexpr (VB) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        cur[e] = __builtin_bit_cast(float, (e & 1) ? (raw[i][e >> 1] & 0xffff0000u) : (raw[i][e >> 1] << 16));
    } else if constexpr (VF) {
#pragma unroll
      for (int e = 0; e < 4; ++e) cur[e] = rawf[i][e];
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) cur[e] = ld1(x + t * xs + c0 + e);
    }
    float res[V];
    uint32_t packed[V / 2 > 0 ? V / 2 : 1];   // bf16 pairs of the output row (bf16, V even)
    if constexpr (sizeof(T) == 2 && V % 2 == 0) {
#pragma unroll
      for (int e = 0; e < V; e += 2) {
        // tap k reads row t + k - (TAPS - 1): win[TAPS - 2 - k], the last tap
        // cur. Each product and sum is rounded on its own (one conversion per
        // value); the first sum, 0 + product, is exact (and turns -0 into +0).
        float a[2];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int k = 0; k < TAPS; ++k) {
            const float sv = k == TAPS - 1 ? cur[e + h] : win[TAPS - 2 - k][e + h];
            const float pr = rnd1_bf16(sv * wt[k][e + h]);
            a[h] = k == 0 ? 0.f + pr : rnd1_bf16(a[h] + pr);
          }
        packed[e / 2] = silu2_bf16(a[0], a[1]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) {
        // tap k reads row t + k - (TAPS - 1): win[TAPS - 2 - k], the last tap cur
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < TAPS; ++k) {
          const float s = k == TAPS - 1 ? cur[e] : win[TAPS - 2 - k][e];
          const float term = rnd<T>(s * wt[k][e]);
          acc = rnd<T>(acc + term);
        }
        res[e] = silu_t<T>(acc);
      }
    }
#pragma unroll
    for (int j = TAPS - 2; j > 0; --j)
#pragma unroll
      for (int e = 0; e < V; ++e) win[j][e] = win[j - 1][e];
#pragma unroll
    for (int e = 0; e < V; ++e) win[0][e] = cur[e];
    if constexpr (VB) {
      *reinterpret_cast<u32x4*>(out + t * os + c0) = (u32x4){packed[0], packed[1], packed[2], packed[3]};
    } else if constexpr (VF) {
      f32x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = res[e];
      *reinterpret_cast<f32x4*>(out + t * os + c0) = v;
    } else if constexpr (sizeof(T) == 2 && V % 2 == 0) {
#pragma unroll
      for (int e = 0; e < V; e += 2) *reinterpret_cast<uint32_t*>(out + t * os + c0 + e) = packed[e / 2];
    } else {
#pragma unroll
      for (int e = 0; e < V; ++e) out[t * os + c0 + e] = (T)res[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Gates: beta = sigmoid(b), g = softplus(a + dt_bias) * neg_a, in f32, each
// step rounded (qwen3_5.rs:494-500, softplus :546-551, candle's sigmoid
// 1 / (1 + exp(-x))).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void gdn_gates_kernel(const T* __restrict__ a, int64_t as,
                                                        const T* __restrict__ bp, int64_t bs,
                                                        const float* __restrict__ dt_bias,
                                                        const float* __restrict__ neg_a, int64_t n_tokens,
                                                        int nv, float* __restrict__ g, float* __restrict__ beta) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n_tokens * nv) return;
  const int64_t t = i / nv;
  const int h = (int)(i - t * nv);
  const float av = ld1(a + t * as + h) + dt_bias[h];
  const float tail = logf(expf(-fabsf(av)) + 1.0f);
  const float sp = fmaxf(av, 0.f) + tail;
  g[i] = sp * neg_a[h];
  const float bv = ld1(bp + t * bs + h);
  beta[i] = __fdiv_rn(1.0f, expf(-bv) + 1.0f);
}

// ---------------------------------------------------------------------------
// The gated delta rule. One workgroup of 8 waves per (value head, text).
// State S [dk <= 128, dv <= 128] f32 in registers: wave w owns value columns
// 16 w .. 16 w + 15; lane l of it holds column 16 w + (l & 15) for key rows
// 32 (l >> 4) .. 32 (l >> 4) + 31, so S^T k and S^T q are 32-term partial
// dot products per lane, completed across the 4 lanes of a column with
// v_permlane16_swap and v_permlane32_swap. The waves never wait on each
// other inside a token: they share only read-only LDS.
//
// Tokens are staged GDN_TB at a time: normalised q and k rows, v, exp(g) and
// beta go to LDS (each wave normalises 2 of the 16 rows with a wave-wide
// reduction); the global loads of the next stage are in flight while the
// current one is computed. Per token and lane: 3 x 32 fused multiply-adds
// (S^T k, the update, S^T q; the decay scales a per-head scalar instead of
// the state); k and q reach the 16 lanes of a row quarter from one LDS
// address (broadcast), one token ahead of their use.
// ---------------------------------------------------------------------------
constexpr int GDN_TB = 16;
constexpr int GDN_DK = 128;
constexpr int GDN_DV = 128;
constexpr int GDN_WAVES = 8;
constexpr int GDN_ROWS = GDN_DK / 4;  // key rows per lane

struct GdnRuleParams {
  const void* mixed;
  int64_t ms;
  const float* g;
  const float* beta;
  int64_t gs;
  float* out;
  int64_t os;
  const int32_t* cu;
  int64_t n;
  int32_t nk, nv, dk, dv;
};

// Sum of x over the 4 lanes l, l ^ 16, l ^ 32, l ^ 48 (the same value on all
// four: each step adds a pair in an order-free way).
__device__ __forceinline__ float quad_sum(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return half_sum(a + b);
}

template <typename T>
__global__ __launch_bounds__(GDN_WAVES * 64) void gdn_rule_kernel(GdnRuleParams p) {
  __shared__ __attribute__((aligned(16))) float s_k[GDN_TB][GDN_DK];
  __shared__ __attribute__((aligned(16))) float s_q[GDN_TB][GDN_DK];
  __shared__ float s_v[GDN_TB][GDN_DV];
  __shared__ float s_dec[GDN_TB];
  __shared__ float s_beta[GDN_TB];

  const int h = blockIdx.x, b = blockIdx.y;
  // cu clamped into [0, n_tokens]: a malformed table gives wrong rows, never an access outside mixed
  const int64_t c0 = p.cu[b], c1 = p.cu[b + 1];
  const int64_t begin = c0 < 0 ? 0 : (c0 > p.n ? p.n : c0);
  const int64_t end = c1 < begin ? begin : (c1 > p.n ? p.n : c1);
  if (end <= begin) return;
  const int kh = h / (p.nv / p.nk);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = 16 * w + (lane & 15), quarter = lane >> 4;
  const T* mx = reinterpret_cast<const T*>(p.mixed);
  const int64_t q_off = (int64_t)kh * p.dk, k_off = (int64_t)(p.nk + kh) * p.dk;
  const int64_t v_off = (int64_t)2 * p.nk * p.dk + (int64_t)h * p.dv;
  const float dk_scale = __fsqrt_rn((float)p.dk);

  // staging registers: wave w stages rows i = w + 8 u; lane holds elements lane, lane + 64
  constexpr int PER_WAVE = GDN_TB / GDN_WAVES;
  float rq[PER_WAVE][2], rk[PER_WAVE][2], rv[PER_WAVE][2], rg[PER_WAVE], rb[PER_WAVE];
  // Loads at clamped (always valid) addresses, masked afterwards: no branch
  // around a load, so no wait before the next one is issued.
  auto fetch = [&](int64_t t0) {
#pragma unroll
    for (int u = 0; u < PER_WAVE; ++u) {
      const int64_t t = t0 + w + GDN_WAVES * u;
      const bool live = t < end;
      const int64_t tc = live ? t : begin;
      const T* row = mx + tc * p.ms;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int r = lane + 64 * e;
        const int rk_ = r < p.dk ? r : 0, rv_ = r < p.dv ? r : 0;
        const float qv = ld1(row + q_off + rk_), kv = ld1(row + k_off + rk_), vv = ld1(row + v_off + rv_);
        rq[u][e] = live && r < p.dk ? qv : 0.f;
        rk[u][e] = live && r < p.dk ? kv : 0.f;
        rv[u][e] = live && r < p.dv ? vv : 0.f;
      }
      const float gv = p.g[tc * p.gs + h], bv = p.beta[tc * p.gs + h];
      rg[u] = live ? gv : 0.f;
      rb[u] = live ? bv : 0.f;
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int u = 0; u < PER_WAVE; ++u) {
      const int i = w + GDN_WAVES * u;
      float sq = rq[u][0] * rq[u][0] + rq[u][1] * rq[u][1];
      float sk = rk[u][0] * rk[u][0] + rk[u][1] * rk[u][1];
      sq = wave_sum(sq);
      sk = wave_sum(sk);
      const float qn = __fsqrt_rn(sq + 1e-6f), kn = __fsqrt_rn(sk + 1e-6f);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        s_q[i][lane + 64 * e] = __fdiv_rn(__fdiv_rn(rq[u][e], qn), dk_scale);
        s_k[i][lane + 64 * e] = __fdiv_rn(rk[u][e], kn);
        s_v[i][lane + 64 * e] = rv[u][e];
      }
      if (lane == 0) {
        s_dec[i] = expf(rg[u]);
        s_beta[i] = rb[u];
      }
    }
  };

  // S = D * Sp: the decays multiply the scalar D instead of the state
  // registers; D is folded back into Sp (Sp *= D, D = 1) before it would
  // drop below 2^-64, so Sp stays within 2^64 of S. D is the same on every
  // lane (it depends on the head's decays only), so the fold is a uniform
  // branch.
  float Sp[GDN_ROWS];
#pragma unroll
  for (int j = 0; j < GDN_ROWS; ++j) Sp[j] = 0.f;
  float D = 1.f;

  auto load_kq = [&](float (&kr)[GDN_ROWS], float (&qr)[GDN_ROWS], int i) {
    const f32x4* k4 = reinterpret_cast<const f32x4*>(&s_k[i][GDN_ROWS * quarter]);
    const f32x4* q4 = reinterpret_cast<const f32x4*>(&s_q[i][GDN_ROWS * quarter]);
#pragma unroll
    for (int j = 0; j < GDN_ROWS / 4; ++j) {
      const f32x4 kv = k4[j], qv = q4[j];
      kr[4 * j] = kv[0]; kr[4 * j + 1] = kv[1]; kr[4 * j + 2] = kv[2]; kr[4 * j + 3] = kv[3];
      qr[4 * j] = qv[0]; qr[4 * j + 1] = qv[1]; qr[4 * j + 2] = qv[2]; qr[4 * j + 3] = qv[3];
    }
  };
  // One token with k, q of row i in (kc, qc); row `next` goes to (kn, qn)
  // meanwhile, so the LDS latency of the next token hides behind this one.
  auto step = [&](float (&kc)[GDN_ROWS], float (&qc)[GDN_ROWS], float (&kn)[GDN_ROWS], float (&qn)[GDN_ROWS],
                  int64_t t, int i, int next) {
    const float dec = s_dec[i], bet = s_beta[i], v = s_v[i][col];
    load_kq(kn, qn, next);
    const float Dn = D * dec;
    if (Dn < 0x1p-64f) {
#pragma unroll
      for (int j = 0; j < GDN_ROWS; ++j) Sp[j] *= Dn;
      D = 1.f;
    } else {
      D = Dn;
    }
    float m0 = 0.f, m1 = 0.f, m2 = 0.f, m3 = 0.f;
#pragma unroll
    for (int j = 0; j < GDN_ROWS; j += 4) {
      m0 = __builtin_fmaf(Sp[j], kc[j], m0);
      m1 = __builtin_fmaf(Sp[j + 1], kc[j + 1], m1);
      m2 = __builtin_fmaf(Sp[j + 2], kc[j + 2], m2);
      m3 = __builtin_fmaf(Sp[j + 3], kc[j + 3], m3);
    }
    const float mem = D * quad_sum((m0 + m1) + (m2 + m3));
    const float u = (v - mem) * bet * __builtin_amdgcn_rcpf(D);
#pragma unroll
    for (int j = 0; j < GDN_ROWS; ++j) Sp[j] = __builtin_fmaf(kc[j], u, Sp[j]);
    float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
#pragma unroll
    for (int j = 0; j < GDN_ROWS; j += 4) {
      o0 = __builtin_fmaf(Sp[j], qc[j], o0);
      o1 = __builtin_fmaf(Sp[j + 1], qc[j + 1], o1);
      o2 = __builtin_fmaf(Sp[j + 2], qc[j + 2], o2);
      o3 = __builtin_fmaf(Sp[j + 3], qc[j + 3], o3);
    }
    const float o = D * quad_sum((o0 + o1) + (o2 + o3));
    if (quarter == 0 && col < p.dv) p.out[t * p.os + (int64_t)h * p.dv + col] = o;
  };

  float kA[GDN_ROWS], qA[GDN_ROWS], kB[GDN_ROWS], qB[GDN_ROWS];
  fetch(begin);
  for (int64_t t0 = begin; t0 < end; t0 += GDN_TB) {
    __syncthreads();  // the previous stage's readers are done
    commit();
    __syncthreads();
    if (t0 + GDN_TB < end) fetch(t0 + GDN_TB);
    const int n = (int)(end - t0 < GDN_TB ? end - t0 : GDN_TB);
    load_kq(kA, qA, 0);
    for (int i = 0; i < n; i += 2) {
      step(kA, qA, kB, qB, t0 + i, i, i + 1 < GDN_TB ? i + 1 : i);
      if (i + 1 < n) step(kB, qB, kA, qA, t0 + i + 1, i + 1, i + 2 < GDN_TB ? i + 2 : i + 1);
    }
  }
}

// ---------------------------------------------------------------------------
// Gated RMSNorm: 32 lanes per (token, head) row of dv <= 128 values; lane l
// holds elements 4 l .. 4 l + 3 (16-byte loads of f32 core when VEC). The
// operation sequence and roundings of late.metal:315-352 (the f32 sum of
// squares is reduced in another order).
// ---------------------------------------------------------------------------
template <typename T, typename TC, bool VEC>
__global__ __launch_bounds__(256) void gdn_gated_norm_kernel(const TC* __restrict__ core, int64_t cs,
                                                             const T* __restrict__ z, int64_t zs,
                                                             const T* __restrict__ w, float eps,
                                                             T* __restrict__ out, int64_t os,
                                                             int64_t n_tokens, int heads, int dv) {
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
  const int l = threadIdx.x & 31;
  const bool live = row < n_tokens * heads;
  const int64_t t = live ? row / heads : 0;
  const int h = live ? (int)(row - t * heads) : 0;
  const TC* cr = core + t * cs + (int64_t)h * dv;
  const T* zr = z + t * zs + (int64_t)h * dv;
  const int c0 = 4 * l;
  float val[4], zv[4];
  if constexpr (VEC) {
    const bool in = live && c0 < dv;
#pragma unroll
    for (int e = 0; e < 4; ++e) { val[e] = 0.f; zv[e] = 0.f; }
    if (in) {
      if constexpr (sizeof(TC) == 4) {
        const f32x4 cv = *reinterpret_cast<const f32x4*>(cr + c0);
#pragma unroll
        for (int e = 0; e < 4; ++e) val[e] = rnd<T>(cv[e]);
      } else {
        const bf16x4 cv = *reinterpret_cast<const bf16x4*>(cr + c0);
#pragma unroll
        for (int e = 0; e < 4; ++e) val[e] = (float)cv[e];
      }
      if constexpr (sizeof(T) == 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(zr + c0);
#pragma unroll
        for (int e = 0; e < 4; ++e) zv[e] = v[e];
      } else {
        const bf16x4 v = *reinterpret_cast<const bf16x4*>(zr + c0);
#pragma unroll
        for (int e = 0; e < 4; ++e) zv[e] = (float)v[e];
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = c0 + e;
      val[e] = (live && c < dv) ? rnd<T>((float)cr[c]) : 0.f;
      zv[e] = (live && c < dv) ? ld1(zr + c) : 0.f;
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) ss += val[e] * val[e];
  ss = group_sum<32>(ss);
  const float inv_dv = __fdiv_rn(1.0f, (float)dv);
  const float scale = __fsqrt_rn(ss * inv_dv + eps);
  if (!live) return;
  T* orow = out + t * os + (int64_t)h * dv;
  float res[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int c = c0 + e < dv ? c0 + e : 0;
    const float normed = rnd<T>(div_t<T>(val[e], scale));
    const float scaled = rnd<T>(normed * ld1(w + c));
    const float sz = div_t<T>(zv[e], 1.0f + exp_t<T>(-zv[e]));
    res[e] = scaled * sz;
  }
  if (VEC) {
    if (c0 < dv) {
      if constexpr (sizeof(T) == 4) {
        f32x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = res[e];
        *reinterpret_cast<f32x4*>(orow + c0) = v;
      } else {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)res[e];
        *reinterpret_cast<bf16x4*>(orow + c0) = v;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c0 + e < dv) orow[c0 + e] = (T)res[e];
  }
}

// ---------------------------------------------------------------------------
// (I + A)^-1 of strictly lower-triangular f32 matrices, size <= 64: one wave
// per matrix, lane j computes column j by forward substitution
//   x[i] = -sum_{k = j .. i-1} A[i, k] x[k]  (x[j] = 1, x[i < j] = 0),
// products and sums rounded in f32 in ascending k (late.metal:64-91). A sits
// in LDS (A[i, k] is one address for every lane: a broadcast) and so does
// the column being built (lane j reads x[k] at xs[k][j]: consecutive banks).
// ---------------------------------------------------------------------------
constexpr int ULI_MAX = 64;

__global__ __launch_bounds__(64) void gdn_unit_lower_inverse_kernel(const float* __restrict__ a, float* __restrict__ out,
                                                                    int size) {
  __shared__ float tile[ULI_MAX][ULI_MAX];
  __shared__ float xs[ULI_MAX][ULI_MAX];
  const int j = threadIdx.x;
  const int64_t m = blockIdx.x;
  const float* src = a + m * size * size;
  for (int i = 0; i < size; ++i)
    if (j < size) tile[i][j] = src[i * size + j];
  __syncthreads();
  if (j >= size) return;
  float* dst = out + m * size * size;
  for (int i = 0; i < size; ++i) {
    float value = 0.f;
    if (i == j) {
      value = 1.f;
    } else if (i > j) {
      float sum = 0.f;
      for (int k = j; k < i; ++k) {
        const float prod = tile[i][k] * xs[k][j];
        sum = sum + prod;
      }
      value = -sum;
    }
    xs[i][j] = value;
    dst[i * size + j] = value;
  }
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename T>
int conv_launch(int64_t n, int n_texts, const int32_t* cu, int channels, int taps, const void* x, int64_t xs,
                const void* w, void* out, int64_t os, hipStream_t st) {
  constexpr int VW = 16 / sizeof(T);
  const bool vec = channels % VW == 0 && xs % VW == 0 && os % VW == 0 && aligned16(x) && aligned16(out);
  const int V = vec ? VW : 1;
  const int64_t runs = (n + CONV_RUN - 1) / CONV_RUN;
  const int64_t threads = runs * (channels / V);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffff) return fail(INL_E_INVALID, "gdn_conv: too many rows x channels");
  const T* xt = static_cast<const T*>(x);
  const T* wt = static_cast<const T*>(w);
  T* ot = static_cast<T*>(out);
  switch (taps * 2 + (vec ? 1 : 0)) {
#define INL_CONV_CASE(K)                                                                                        \
  case 2 * K + 1:                                                                                               \
    hipLaunchKernelGGL((gdn_conv_kernel<T, VW, K>), dim3((unsigned)blocks), dim3(256), 0, st, xt, xs, cu, n_texts, \
                       n, channels, wt, ot, os);                                                                \
    break;                                                                                                      \
  case 2 * K:                                                                                                   \
    hipLaunchKernelGGL((gdn_conv_kernel<T, 1, K>), dim3((unsigned)blocks), dim3(256), 0, st, xt, xs, cu, n_texts,  \
                       n, channels, wt, ot, os);                                                                \
    break;
    INL_CONV_CASE(1)
    INL_CONV_CASE(2)
    INL_CONV_CASE(3)
    INL_CONV_CASE(4)
    INL_CONV_CASE(5)
    INL_CONV_CASE(6)
    INL_CONV_CASE(7)
    INL_CONV_CASE(8)
#undef INL_CONV_CASE
    default:
      return fail(INL_E_INVALID, "gdn_conv: 1 <= taps <= 8");
  }
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

}  // namespace

}  // namespace inl

using namespace inl;

extern "C" int inl_gdn_conv_fwd(int64_t n_tokens, int32_t n_texts, const int32_t* cu_seqlens, int32_t channels,
                                int32_t taps, int32_t dtype, const void* x, int64_t x_stride, const void* weight,
                                void* out, int64_t out_stride, void* stream) {
  if (n_tokens < 0 || n_texts < 0 || channels <= 0 || taps < 1 || taps > CONV_MAX_TAPS || !dtype_ok(dtype))
    return fail(INL_E_INVALID, "gdn_conv: need n_tokens >= 0, channels > 0, 1 <= taps <= 8, dtype f32 or bf16");
  if (n_tokens == 0) return INL_OK;
  if (n_texts < 1 || !cu_seqlens || !x || !weight || !out)
    return fail(INL_E_INVALID, "gdn_conv: null pointer or no texts");
  const int64_t xs = x_stride ? x_stride : channels, os = out_stride ? out_stride : channels;
  if (xs < channels || os < channels) return fail(INL_E_INVALID, "gdn_conv: stride shorter than a row");
  hipStream_t st = as_stream(stream);
  return dtype == INL_BF16 ? conv_launch<bf16>(n_tokens, n_texts, cu_seqlens, channels, taps, x, xs, weight, out, os, st)
                           : conv_launch<float>(n_tokens, n_texts, cu_seqlens, channels, taps, x, xs, weight, out, os, st);
}

extern "C" int inl_gdn_gates_fwd(int64_t n_tokens, int32_t value_heads, int32_t dtype, const void* a,
                                 int64_t a_stride, const void* b, int64_t b_stride, const float* dt_bias,
                                 const float* neg_a, float* g, float* beta, void* stream) {
  if (n_tokens < 0 || value_heads <= 0 || !dtype_ok(dtype))
    return fail(INL_E_INVALID, "gdn_gates: need n_tokens >= 0, value_heads > 0, dtype f32 or bf16");
  if (n_tokens == 0) return INL_OK;
  if (!a || !b || !dt_bias || !neg_a || !g || !beta) return fail(INL_E_INVALID, "gdn_gates: null pointer");
  const int64_t as = a_stride ? a_stride : value_heads, bs = b_stride ? b_stride : value_heads;
  if (as < value_heads || bs < value_heads) return fail(INL_E_INVALID, "gdn_gates: stride shorter than a row");
  const int64_t total = n_tokens * value_heads;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffff) return fail(INL_E_INVALID, "gdn_gates: too many rows");
  hipStream_t st = as_stream(stream);
  if (dtype == INL_BF16)
    hipLaunchKernelGGL(gdn_gates_kernel<bf16>, dim3((unsigned)blocks), dim3(256), 0, st,
                       static_cast<const bf16*>(a), as, static_cast<const bf16*>(b), bs, dt_bias, neg_a, n_tokens,
                       value_heads, g, beta);
  else
    hipLaunchKernelGGL(gdn_gates_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st,
                       static_cast<const float*>(a), as, static_cast<const float*>(b), bs, dt_bias, neg_a, n_tokens,
                       value_heads, g, beta);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

extern "C" int inl_gdn_rule_fwd(int64_t n_tokens, int32_t n_texts, const int32_t* cu_seqlens, int32_t key_heads,
                                int32_t value_heads, int32_t key_dim, int32_t value_dim, int32_t dtype,
                                const void* mixed, int64_t mixed_stride, const float* g, const float* beta,
                                int64_t gate_stride, float* out, int64_t out_stride, void* stream) {
  if (n_tokens < 0 || n_texts < 0 || key_heads <= 0 || value_heads <= 0 || value_heads % key_heads != 0 ||
      key_dim < 1 || key_dim > GDN_DK || value_dim < 1 || value_dim > GDN_DV || !dtype_ok(dtype))
    return fail(INL_E_INVALID,
                "gdn_rule: need value_heads a multiple of key_heads, 1 <= key_dim, value_dim <= 128, dtype f32 or bf16");
  if (n_tokens == 0 || n_texts == 0) return INL_OK;
  if (!cu_seqlens || !mixed || !g || !beta || !out) return fail(INL_E_INVALID, "gdn_rule: null pointer");
  if (n_texts > 65535) return fail(INL_E_INVALID, "gdn_rule: at most 65535 texts per call");
  const int64_t channels = 2LL * key_heads * key_dim + (int64_t)value_heads * value_dim;
  GdnRuleParams p;
  p.mixed = mixed;
  p.ms = mixed_stride ? mixed_stride : channels;
  p.g = g;
  p.beta = beta;
  p.gs = gate_stride ? gate_stride : value_heads;
  p.out = out;
  p.os = out_stride ? out_stride : (int64_t)value_heads * value_dim;
  if (p.ms < channels || p.gs < value_heads || p.os < (int64_t)value_heads * value_dim)
    return fail(INL_E_INVALID, "gdn_rule: stride shorter than a row");
  p.cu = cu_seqlens;
  p.n = n_tokens;
  p.nk = key_heads;
  p.nv = value_heads;
  p.dk = key_dim;
  p.dv = value_dim;
  hipStream_t st = as_stream(stream);
  const dim3 grid((unsigned)value_heads, (unsigned)n_texts);
  if (dtype == INL_BF16) hipLaunchKernelGGL(gdn_rule_kernel<bf16>, grid, dim3(GDN_WAVES * 64), 0, st, p);
  else hipLaunchKernelGGL(gdn_rule_kernel<float>, grid, dim3(GDN_WAVES * 64), 0, st, p);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

extern "C" int inl_gdn_gated_norm_fwd(int64_t n_tokens, int32_t heads, int32_t value_dim, int32_t dtype,
                                      int32_t core_dtype, const void* core, int64_t core_stride, const void* z,
                                      int64_t z_stride, const void* weight, float eps, void* out,
                                      int64_t out_stride, void* stream) {
  if (n_tokens < 0 || heads <= 0 || value_dim < 1 || value_dim > GDN_DV || !dtype_ok(dtype) ||
      !(core_dtype == INL_F32 || core_dtype == dtype))
    return fail(INL_E_INVALID, "gdn_gated_norm: need 1 <= value_dim <= 128, dtype f32 or bf16, core in f32 or dtype");
  if (n_tokens == 0) return INL_OK;
  if (!core || !z || !weight || !out) return fail(INL_E_INVALID, "gdn_gated_norm: null pointer");
  const int64_t row = (int64_t)heads * value_dim;
  const int64_t cs = core_stride ? core_stride : row, zs = z_stride ? z_stride : row,
                os = out_stride ? out_stride : row;
  if (cs < row || zs < row || os < row) return fail(INL_E_INVALID, "gdn_gated_norm: stride shorter than a row");
  const int64_t rows = n_tokens * heads;
  const int64_t blocks = (rows * 32 + 255) / 256;
  if (blocks > 0x7fffffff) return fail(INL_E_INVALID, "gdn_gated_norm: too many rows");
  hipStream_t st = as_stream(stream);
  const dim3 grid((unsigned)blocks);
  const int csz = core_dtype == INL_F32 ? 4 : 2, tsz = dtype_size(dtype);
  const bool vec = value_dim % 4 == 0 && (cs * csz) % 16 == 0 && aligned16(core) && (zs * tsz) % 8 == 0 &&
                   (os * tsz) % 8 == 0 && (reinterpret_cast<uintptr_t>(z) & 7) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) & 7) == 0 && ((int64_t)value_dim * csz) % 16 == 0;
#define INL_NORM_LAUNCH(T, TC)                                                                                     \
  if (vec)                                                                                                         \
    hipLaunchKernelGGL((gdn_gated_norm_kernel<T, TC, true>), grid, dim3(256), 0, st, static_cast<const TC*>(core), \
                       cs, static_cast<const T*>(z), zs, static_cast<const T*>(weight), eps, static_cast<T*>(out), os, \
                       n_tokens, heads, value_dim);                                                                \
  else                                                                                                             \
    hipLaunchKernelGGL((gdn_gated_norm_kernel<T, TC, false>), grid, dim3(256), 0, st, static_cast<const TC*>(core), \
                       cs, static_cast<const T*>(z), zs, static_cast<const T*>(weight), eps, static_cast<T*>(out), os, \
                       n_tokens, heads, value_dim);
  if (dtype == INL_BF16) {
    if (core_dtype == INL_F32) {
      INL_NORM_LAUNCH(bf16, float)
    } else {
      INL_NORM_LAUNCH(bf16, bf16)
    }
  } else {
    INL_NORM_LAUNCH(float, float)
  }
#undef INL_NORM_LAUNCH
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}

extern "C" int inl_gdn_unit_lower_inverse_fwd(int64_t n, int32_t size, const float* a, float* out, void* stream) {
  if (n < 0 || size < 1 || size > ULI_MAX)
    return fail(INL_E_INVALID, "gdn_unit_lower_inverse: need n >= 0 and 1 <= size <= 64");
  if (n == 0) return INL_OK;
  if (!a || !out) return fail(INL_E_INVALID, "gdn_unit_lower_inverse: null pointer");
  if (n > 0x7fffffff) return fail(INL_E_INVALID, "gdn_unit_lower_inverse: too many matrices");
  hipLaunchKernelGGL(gdn_unit_lower_inverse_kernel, dim3((unsigned)n), dim3(64), 0, as_stream(stream), a, out, size);
  INL_HIP_TRY(hipGetLastError());
  return INL_OK;
}
