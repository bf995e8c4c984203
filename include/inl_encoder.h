/*
 * inl_encoder.h - C ABI of the layer ops around the attention path and of a
 * whole-encoder runner, on one MI355X (gfx950).
 *
 * The reference runs an encoder's projections, norms and MLP as candle ops
 * (crates/inl-text/src/qwen3/mod.rs:72-116,227-297,339-358). The calls below
 * are their GPU counterparts, so that an engine's forward runs on the device
 * end to end: the GEMMs on hipBLASLt (inl_linear_fwd), the element-wise ops
 * on the library's own kernels. Conventions are those of inl_hip.h (device
 * pointers unless named `_host`, int status + inl_last_error(), work on the
 * caller's stream, the caller owns every buffer).
 */
#ifndef INL_ENCODER_H
#define INL_ENCODER_H

#include <stddef.h>
#include <stdint.h>

#include "inl_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * Layer ops
 * --------------------------------------------------------------------- */

/* y[m, n] = alpha * x[m, k] . w[n, k]^T + beta * y: a bias-free candle
 * `Linear` (qwen3/mod.rs:99-104, q/k/v/o projections :188-209, gate/up/down
 * :96-106) with its row-major [out, in] weight. beta = 1 accumulates into y,
 * which is how a residual addition (qwen3/mod.rs:291-296) folds into the
 * o_proj and down_proj GEMMs. dtypes: f32 -> f32, bf16 -> bf16, bf16 -> f32.
 * Strides are elements between rows (0 = packed). `workspace` (device, may be
 * NULL with 0 bytes) lets hipBLASLt pick kernels that need scratch; size it
 * with inl_linear_workspace_size. Runs hipBLASLt. Row counts m fall in
 * power-of-two buckets ((2^(b-1), 2^b], m <= 64 in one): per device, shape
 * (n, k, strides, dtypes, beta != 0, workspace) and bucket, the first call
 * queries the heuristic and, unless `stream` is capturing a graph, times up
 * to 16 of its candidates on the call's operands (into a scratch output it
 * allocates and frees; y is not touched) and keeps the fastest. That call
 * synchronises the stream. Any other m of the bucket reuses the choice once
 * hipBLASLt confirms it supports that m (host-side only: no allocation, no
 * synchronisation, no device work besides the GEMM); the per-m layouts are
 * cached, the oldest of 512 evicted first. */
int inl_linear_workspace_size(size_t* bytes);
/* Diagnostics of inl_linear_fwd's cache (process-wide, all devices): timing
 * passes run so far, (shape, bucket) choices held, exact-m entries held. Any
 * out-pointer may be NULL. No reference counterpart. */
int inl_linear_stats(int64_t* tunings, int64_t* buckets, int64_t* cached_shapes);
int inl_linear_fwd(int64_t m, int64_t n, int64_t k, int32_t in_dtype,
                   const void* x, int64_t x_stride, const void* w,
                   int64_t w_stride, int32_t out_dtype, void* y,
                   int64_t y_stride, float alpha, float beta, void* workspace,
                   size_t workspace_bytes, void* stream);

/* y = alpha * x . w^T + beta * y on the matrix cores, bf16 x [m, k] and
 * w [n, k] rows (row strides in elements, 0 = packed), f32 accumulation,
 * y [m, n] rows in out_dtype (f32 or bf16). The same bias-free Linear as
 * inl_linear_fwd (candle_nn::Linear through linear_no_bias,
 * crates/inl-text/src/qwen3/mod.rs:99-104, crates/inl-text/src/gemma2.rs:
 * 233-283), as one hand-written kernel: no workspace, no allocation, no
 * tuning, no synchronisation, for every m (graph-capturable). k a multiple
 * of 32, n and the strides multiples of 8, pointers 16-byte aligned. */
int inl_gemm_bf16_fwd(int64_t m, int64_t n, int64_t k, const void* x,
                      int64_t x_stride, const void* w, int64_t w_stride,
                      int32_t out_dtype, void* y, int64_t y_stride,
                      float alpha, float beta, void* stream);

/* The same GEMM with a gated epilogue, for the GEGLU gates of EmbeddingGemma
 * 2 (crates/inl-text/src/gemma2.rs:249-254 Mlp::forward, :279-283 the
 * per-layer-input gate), gelu_tanh(v) = v/2 (1 + tanh(sqrt(2/pi)(v + 0.044715
 * v^3))) in f32 on the f32 products:
 *   INL_GATE_GEGLU:    w [2n, k] = gate rows then up rows (the stacked
 *                      gate/up projection);
 *                      y[m, c] = gelu_tanh(x . w[c]) * (x . w[n + c])
 *   INL_GATE_GELU_MUL: w [n, k]; mul [m, n] bf16 rows of mul_stride;
 *                      y[m, c] = gelu_tanh(x . w[c]) * mul[m, c]
 * The gate and up products never reach memory. Limits as inl_gemm_bf16_fwd
 * (mul 8-byte aligned, mul_stride a multiple of 4). */
#define INL_GATE_GEGLU 1
#define INL_GATE_GELU_MUL 2
int inl_gemm_bf16_gated_fwd(int64_t m, int64_t n, int64_t k, const void* x,
                            int64_t x_stride, const void* w, int64_t w_stride,
                            int32_t mode, const void* mul, int64_t mul_stride,
                            int32_t out_dtype, void* y, int64_t y_stride,
                            void* stream);

/* out[t, :] = f32(table[ids[t], :]): the token embedding (candle Embedding,
 * qwen3/mod.rs:322-323,350) into an f32 residual stream. ids are device
 * int32; an id outside [0, vocab) yields a NaN row (check ids first). */
int inl_embed_fwd(int64_t n_tokens, const int32_t* ids, const void* table,
                  int64_t vocab, int32_t hidden, int32_t dtype, float* out,
                  int64_t out_stride, void* stream);

/* y = x / sqrt(mean(x^2) + eps) * weight per row of an f32 stream x, written
 * in out_dtype: the pre-norm RMSNorm of qwen3/mod.rs:72-90 (input_layernorm,
 * post_attention_layernorm :287-295). weight NULL = ones. dim and x_stride
 * multiples of 4, x 16-byte aligned. */
int inl_rms_norm_rows_fwd(int64_t rows, int32_t dim, const float* x,
                          int64_t x_stride, const void* weight,
                          int32_t weight_dtype, float eps, int32_t out_dtype,
                          void* y, int64_t y_stride, void* stream);

/* out[t, i] = silu(gate_up[t, i]) * gate_up[t, intermediate + i], silu(g) =
 * g / (1 + exp(-g)) in f32: the MLP gate of qwen3/mod.rs:109-116 over a fused
 * gate/up projection output (gate rows first). Sizes and strides 16-byte
 * multiples. */
int inl_swiglu_fwd(int64_t rows, int32_t intermediate, int32_t dtype,
                   const void* gate_up, int64_t gu_stride, void* out,
                   int64_t out_stride, void* stream);

/* ------------------------------------------------------------------------
 * Fused SPLADE decoder + max (crates/inl-sparse/src/modernbert.rs:657-662
 * `project`'s bias-free decoder, :806-872 `pool_states`'s per-row max):
 *   out[r, v] = max over p in [offs_host[r], offs_host[r+1]) of
 *               head[p, :] . w_dec[v, :]        (f32; -inf without positions)
 * for the packed MLM-head outputs of every speaking position (head
 * [S, hidden], bf16) and the decoder weight w_dec [vocab, hidden] (bf16),
 * without writing the [S, vocab] logits. Feed `out` to inl_splade_finish_fwd
 * (inl_hip.h) for the bias, shift, relu, log1p, mask and canonical fold.
 * hidden a multiple of 32; strides in elements, 16-byte multiples. The
 * workspace (device, 16-byte aligned) holds the launch schedule. The max is
 * taken over f32 products accumulated in f32 on the matrix cores: for given
 * bf16 inputs it differs from a sequential f32 sum only in rounding.
 * --------------------------------------------------------------------- */
int inl_splade_decoder_workspace_size(int32_t rows, int32_t vocab, size_t* bytes);
int inl_splade_decoder_max_fwd(int32_t rows, const int32_t* offs_host,
                               const void* head, int64_t head_stride,
                               int32_t hidden, const void* w_dec,
                               int64_t w_stride, int32_t vocab, int32_t dtype,
                               float* out, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Qwen3 encoder runner: the GPU counterpart of Qwen3Model::forward_last and
 * Qwen3Embedder::embed (crates/inl-text/src/qwen3/mod.rs:339-358,438-470)
 * over packed texts (each text's last row pooled; positions restart at 0 per
 * text, as in the reference's left-padded batch). The weights stay the
 * caller's; two projections are fused by stacking rows:
 *   qkv_proj:     [(heads + 2 kv_heads) * head_dim, hidden] = q_proj rows,
 *                 then k_proj rows, then v_proj rows;
 *   gate_up_proj: [2 * intermediate, hidden] = gate_proj rows, then up_proj.
 * All weights are in `dtype` (INL_F32 or INL_BF16). The residual stream is
 * f32 in both modes; GEMM inputs and attention run in `dtype`.
 * --------------------------------------------------------------------- */
typedef struct inl_qwen3_config {
  int32_t vocab;
  int32_t hidden;
  int32_t intermediate;
  int32_t layers;
  int32_t heads;
  int32_t kv_heads;
  int32_t head_dim;       /* 128 for the benchmark shape */
  float eps;              /* rms_norm_eps */
  double rope_theta;
  int32_t max_positions;  /* longest text the RoPE table covers */
  int32_t dtype;          /* enum inl_dtype of the weights and activations */
  int32_t attn_flags;     /* INL_ATTN_* (INL_ATTN_PV_BF16 for V beyond fp16) */
} inl_qwen3_config;

typedef struct inl_qwen3_layer_weights {
  const void* qkv_proj;
  const void* o_proj;         /* [hidden, heads * head_dim] */
  const void* gate_up_proj;
  const void* down_proj;      /* [hidden, intermediate] */
  const void* q_norm;         /* [head_dim] */
  const void* k_norm;         /* [head_dim] */
  const void* input_norm;     /* [hidden] */
  const void* post_attention_norm; /* [hidden] */
} inl_qwen3_layer_weights;

typedef struct inl_qwen3 inl_qwen3;

/* Keeps the weight pointers (and copies the layer table); builds the RoPE
 * tables (f64 angles, qwen3/mod.rs:131-153) and an f32 copy of the final
 * norm on the current device - the only allocations the runner makes. */
int inl_qwen3_create(const inl_qwen3_config* cfg, const void* embed_tokens,
                     const inl_qwen3_layer_weights* layers,
                     const void* final_norm, inl_qwen3** enc);
int inl_qwen3_destroy(inl_qwen3* enc);

/* Device workspace one encode of these texts needs (activations, the
 * attention schedule, the GEMM workspace). */
int inl_qwen3_workspace_size(const inl_qwen3* enc, int32_t n_texts,
                             const int32_t* cu_seqlens_host, size_t* bytes);

/* embeddings[b, :] (device f32 [n_texts, hidden]) = L2-normalised final
 * RMSNorm of text b's last row (+1e-12 inside the square root,
 * qwen3/mod.rs:468). ids_host: [cu_seqlens_host[n_texts]] token ids, checked
 * against vocab on the host. Texts of length 0 are refused, as the
 * reference refuses an empty tokenisation (qwen3/mod.rs:446-448).
 * The batch (ids, positions, offsets, the attention schedule) is uploaded
 * on `stream` from the encoder's pinned staging buffer (held until those
 * copies complete; it grows on the first call that needs more), then the layers
 * run. With graphs on (the default), the launch sequence of a batch shape -
 * the same device, cu_seqlens_host, workspace and embeddings pointer - is
 * captured on its second call and replayed from the third on (the first
 * runs eagerly). Calls on one encoder are serialised by a lock; the
 * encoder keeps the graph of one shape at a time. */
int inl_qwen3_encode(inl_qwen3* enc, int32_t n_texts,
                     const int32_t* cu_seqlens_host, const int32_t* ids_host,
                     float* embeddings, void* workspace, size_t workspace_bytes,
                     void* stream);

/* Turns the launch-sequence graph of inl_qwen3_encode on (enable != 0, the
 * default) or off, and drops the graph held. No counterpart in the
 * reference, whose candle forward issues every op eagerly. */
int inl_qwen3_set_graphs(inl_qwen3* enc, int32_t enable);
/* *enabled: graphs are on (they turn off by themselves if capture is not
 * possible or a captured graph holds a memset); *held: a graph of the last
 * batch shape is instantiated and will be launched by the next call of
 * that shape. */
int inl_qwen3_graph_info(inl_qwen3* enc, int32_t* enabled, int32_t* held);

/* ------------------------------------------------------------------------
 * EmbeddingGemma 2 text-tower runner: the GPU counterpart of
 * Gemma2Model::forward_pooled (crates/inl-text/src/gemma2.rs:612-662, the
 * layer of :473-494, the attention of :381-441, the MLP of :249-254 and the
 * per-layer-input block of :279-283) over packed texts: bidirectional
 * attention, sliding layers windowed to |q - k| <= sliding_window, mean
 * pooling, the embedding projection and L2, then optionally the Matryoshka
 * truncate-and-renormalise of crates/inl-text/src/native.rs:822-830.
 * As for Qwen3 the weights stay the caller's, in `dtype`, with
 *   qkv_proj:     [(heads + 2 kv_heads) * head_dim, hidden] = q, k, v rows;
 *   gate_up_proj: [2 * intermediate, hidden] = gate rows, then up rows.
 * The residual stream is f32; GEMM inputs and attention run in `dtype`.
 * --------------------------------------------------------------------- */
typedef struct inl_gemma2_config {
  int32_t vocab;
  int32_t hidden;
  int32_t intermediate;
  int32_t layers;
  int32_t heads;
  int32_t kv_heads;        /* default; a layer may override it */
  int32_t head_dim;        /* default; a layer may override it */
  int32_t ple_dim;         /* hidden_size_per_layer_input */
  int32_t embedding_dim;   /* rows of embedding_projection */
  int32_t sliding_window;  /* inclusive radius of the sliding layers */
  float eps;               /* rms_norm_eps */
  double theta_sliding;    /* rope_theta of sliding_attention layers */
  double theta_full;       /* rope_theta of full_attention layers */
  int32_t max_positions;   /* longest text the RoPE tables cover */
  int32_t dtype;           /* enum inl_dtype of the weights and activations */
  int32_t attn_flags;      /* INL_ATTN_* */
} inl_gemma2_config;

typedef struct inl_gemma2_layer_weights {
  int32_t full;            /* 1 = full_attention, 0 = sliding_attention */
  int32_t head_dim;        /* 0 = the config's (per_layer_config override) */
  int32_t kv_heads;        /* 0 = the config's */
  const void* qkv_proj;
  const void* o_proj;      /* [hidden, heads * head_dim] */
  const void* gate_up_proj;
  const void* down_proj;   /* [hidden, intermediate] */
  const void* q_norm;      /* [head_dim] */
  const void* k_norm;      /* [head_dim] */
  const void* input_norm;              /* [hidden] */
  const void* post_attention_norm;     /* [hidden] */
  const void* pre_feedforward_norm;    /* [hidden] */
  const void* post_feedforward_norm;   /* [hidden] */
  const void* ple_input_gate;          /* [ple_dim, hidden] */
  const void* ple_projection;          /* [hidden, ple_dim] */
  const void* ple_post_norm;           /* [hidden] */
  const void* layer_scalar;            /* [1] */
} inl_gemma2_layer_weights;

typedef struct inl_gemma2 inl_gemma2;

/* Keeps the weight pointers; builds the two RoPE tables (f64 angles,
 * gemma2.rs:292-315) and f32 copies of the layer scalars on the current
 * device - the only allocations the runner makes. ple_model_projection:
 * [layers * ple_dim, hidden]; ple_norm: [ple_dim]; final_norm: [hidden];
 * embedding_projection: [embedding_dim, hidden]. */
int inl_gemma2_create(const inl_gemma2_config* cfg, const void* embed_tokens,
                      const inl_gemma2_layer_weights* layers,
                      const void* ple_model_projection, const void* ple_norm,
                      const void* final_norm, const void* embedding_projection,
                      inl_gemma2** enc);
int inl_gemma2_destroy(inl_gemma2* enc);

/* Device workspace one encode of these texts needs. */
int inl_gemma2_workspace_size(const inl_gemma2* enc, int32_t n_texts,
                              const int32_t* cu_seqlens_host, size_t* bytes);

/* embeddings (device f32 [n_texts, out_dim]) = the L2-normalised projection
 * of each text's mean final hidden state (1e-12 inside the square root,
 * gemma2.rs:660-661); out_dim < embedding_dim keeps the first out_dim
 * values and normalises them again (Matryoshka; a zero row stays zero).
 * ids_host: [cu_seqlens_host[n_texts]] token ids, checked against vocab.
 * Texts of length 0 are refused. Launches run eagerly on `stream`. */
int inl_gemma2_encode(inl_gemma2* enc, int32_t n_texts,
                      const int32_t* cu_seqlens_host, const int32_t* ids_host,
                      int32_t out_dim, float* embeddings, void* workspace,
                      size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* INL_ENCODER_H */
