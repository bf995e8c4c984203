/*
 * inl_gdn.h - C ABI of the gated-delta-net (linear attention) ops of the
 * pplx-late Qwen3.5 tower, on one MI355X (gfx950).
 *
 * The reference runs these as four Metal kernels behind candle custom ops
 * (crates/inl-late/src/metal.rs, crates/inl-late/src/late.metal) inside
 * GatedDeltaNet::forward (crates/inl-late/src/qwen3_5.rs:481-545). Here texts
 * are packed: rows of every text follow each other, `cu_seqlens` (device
 * int32, n_texts + 1 entries, cu[0] = 0, nondecreasing) marks where each text
 * starts, and each text starts from a zero state, as each right-padded row
 * of the reference's batch does (its rule and convolution are causal, so the
 * padding never reaches a real token, qwen3_5.rs:1-7). Conventions are those
 * of inl_hip.h: device pointers, int status + inl_last_error(), work on the
 * caller's stream, the caller owns every buffer. dtypes: INL_F32, INL_BF16.
 * Strides are elements between consecutive tokens (0 = packed). The kernels
 * read cu_seqlens on the device and clamp its entries into [0, n_tokens], so
 * a table that does not end at n_tokens gives wrong rows but no access
 * outside the buffers.
 */
#ifndef INL_GDN_H
#define INL_GDN_H

#include <stddef.h>
#include <stdint.h>

#include "inl_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* out[t, c] = silu(sum_k x[t + k - (taps - 1), c] * weight[c, k]), rows
 * before the text's first row read as zero: the depthwise causal convolution
 * fused with its silu (metal.rs:119-143 `causal_conv`, kernel late.metal:
 * 104-154; the candle form GatedDeltaNet::causal_conv, qwen3_5.rs:463-479).
 * Every product, sum and silu step rounds in `dtype`, in tap order, as the
 * reference's kernel does. x, out: [n_tokens, channels]; weight: [channels,
 * taps] in `dtype`; 1 <= taps <= 8. */
int inl_gdn_conv_fwd(int64_t n_tokens, int32_t n_texts, const int32_t* cu_seqlens,
                     int32_t channels, int32_t taps, int32_t dtype,
                     const void* x, int64_t x_stride, const void* weight,
                     void* out, int64_t out_stride, void* stream);

/* The gates of the rule (qwen3_5.rs:494-500): for value head h,
 *   beta[t, h] = sigmoid(b[t, h]),
 *   g[t, h]    = softplus(a[t, h] + dt_bias[h]) * neg_a[h],
 * softplus(x) = relu(x) + log(1 + exp(-|x|)) (qwen3_5.rs:546-551), in f32.
 * a, b: the in_proj_a / in_proj_b outputs [n_tokens, value_heads] in
 * `dtype`; dt_bias, neg_a (= -exp(A_log), qwen3_5.rs:452): f32
 * [value_heads]; g, beta: f32 [n_tokens, value_heads], packed. */
int inl_gdn_gates_fwd(int64_t n_tokens, int32_t value_heads, int32_t dtype,
                      const void* a, int64_t a_stride, const void* b,
                      int64_t b_stride, const float* dt_bias,
                      const float* neg_a, float* g, float* beta, void* stream);

/* The gated delta rule, per text and value head h, token by token
 * (metal.rs:145-190 `recurrent_delta`, kernel late.metal:156-291; the
 * chunked form qwen3_5.rs:598-728 computes the same function):
 *   q = l2norm(q_kh) / sqrt(dk), k = l2norm(k_kh), kh = h / (nv / nk),
 *   l2norm(x) = x / sqrt(sum(x^2) + 1e-6),
 *   S = S * exp(g); delta = (v - S^T k) * beta; S = S + k delta^T;
 *   out = S^T q,                    S: [dk, dv] f32, zero at each text start.
 * mixed: [n_tokens, 2 nk dk + nv dv] in `dtype` (the convolution's output:
 * q heads, k heads, v heads); g, beta: f32 [n_tokens, nv] with `gate_stride`;
 * out: f32 [n_tokens, nv, dv] with `out_stride` elements between tokens.
 * nv a multiple of nk; 1 <= dk, dv <= 128. The state stays in registers,
 * f32, with fused multiply-adds (the reference's kernel rounds each product
 * and sum; the difference is rounding only). */
int inl_gdn_rule_fwd(int64_t n_tokens, int32_t n_texts, const int32_t* cu_seqlens,
                     int32_t key_heads, int32_t value_heads, int32_t key_dim,
                     int32_t value_dim, int32_t dtype, const void* mixed,
                     int64_t mixed_stride, const float* g, const float* beta,
                     int64_t gate_stride, float* out, int64_t out_stride,
                     void* stream);

/* The gated RMSNorm after the rule, per (token, head) row of value_dim
 * (metal.rs:190-215 `gated_norm`, kernel late.metal:294-352; candle form
 * qwen3_5.rs:526-541):
 *   c = dtype(core); var = sum(c^2) * (1 / dv);
 *   n = dtype(c / sqrt(var + eps)); s = dtype(n * weight);
 *   out = dtype(f32(s) * silu_f32(z)).
 * core: [n_tokens, heads, dv] in `core_dtype` (INL_F32 = the rule's output,
 * rounded to `dtype` first, as qwen3_5.rs:530 does; or `dtype`); z, out:
 * [n_tokens, heads, dv] in `dtype`; weight: [dv] in `dtype`; dv <= 128. */
int inl_gdn_gated_norm_fwd(int64_t n_tokens, int32_t heads, int32_t value_dim,
                           int32_t dtype, int32_t core_dtype, const void* core,
                           int64_t core_stride, const void* z, int64_t z_stride,
                           const void* weight, float eps, void* out,
                           int64_t out_stride, void* stream);

/* out[m] = (I + a[m])^-1 for n strictly lower-triangular f32 [size, size]
 * matrices (contiguous), by forward substitution per column, each product
 * and sum rounded in f32 in the reference's order (metal.rs:95-117
 * `unit_lower_inverse`, kernel late.metal:31-92; the chunked rule's solve,
 * qwen3_5.rs:734-773). 1 <= size <= 64 (the reference takes powers of two). */
int inl_gdn_unit_lower_inverse_fwd(int64_t n, int32_t size, const float* a,
                                   float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INL_GDN_H */
