/*
 * inl_hip.h - C ABI of the MI355X (gfx950) encoder-attention path.
 *
 * The library exports plain C functions over device pointers and sizes, so
 * that im-not-llm's Rust engines can bind it over FFI and wrap it as a candle
 * custom op. Every pointer named `q`, `k`, `v`, `out`, `x`, `y`, `hidden`,
 * `logits`, `pooled`, `cos`, `sin`, `weight`, `bias`, `canonical`, `rows`,
 * `cu`, `offs` is a device pointer; names ending in `_host` are host
 * pointers. Work is enqueued on `stream` (a hipStream_t; NULL = the null
 * stream) and is asynchronous unless a function says otherwise.
 *
 * Errors: every function returns 0 on success and a negative INL_E_* code
 * otherwise; inl_last_error() returns the message of the calling thread's
 * last failure. The caller owns every buffer. Calls on one stream need no
 * locking; calls may come from several host threads.
 *
 * Packed layout: texts are stored back to back, token-major. Text b owns rows
 * [cu_seqlens[b], cu_seqlens[b+1]) of every packed tensor; a token row holds
 * all heads contiguously (`heads * head_dim` elements), and consecutive token
 * rows are `*_row_stride` elements apart (>= heads * head_dim), so the q, k
 * and v slices of one fused QKV projection output can be passed without a
 * copy. Attention never crosses texts, and RoPE positions restart at 0 for
 * every text (the packing rule of the reference's
 * crates/inl-ane/src/layout.rs:1-7,391-415).
 */
#ifndef INL_HIP_H
#define INL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define INL_HIP_ABI_VERSION 2

enum inl_status {
  INL_OK = 0,
  INL_E_INVALID = -1,     /* bad argument (shape, dtype, alignment, range) */
  INL_E_UNSUPPORTED = -2, /* valid request this build has no kernel for */
  INL_E_HIP = -3,         /* a HIP runtime call failed */
  INL_E_NOMEM = -4        /* a host or device allocation failed */
};

enum inl_dtype { INL_F32 = 0, INL_BF16 = 1 };

/* ------------------------------------------------------------------------
 * Attention
 *
 * Replaces the attention call of every encoder engine:
 *   - crates/inl-core/src/attention.rs:215-234 `attend` (Qwen3 causal GQA:
 *     causal=1, window=-1, scale=head_dim^-0.5), with its Eager/Tiled/
 *     CpuFlash backends (:236-315);
 *   - crates/inl-text/src/gemma2.rs:414-441 (EmbeddingGemma 2: causal=0,
 *     scale=1, window=sliding_window for sliding layers, -1 for full);
 *   - crates/inl-sparse/src/modernbert.rs:366-401 (ModernBERT: causal=0,
 *     scale=head_dim^-0.5, window=local_attention/2 on local layers);
 *   - crates/inl-late/src/qwen3_5.rs:364-407 (Qwen3.5 full attention:
 *     causal=is_causal, scale=head_dim^-0.5);
 *   - crates/inl-vision/src/vision.rs:226-259 (vision tower: causal=0,
 *     scale=1, window=-1).
 * The reference's padded batches and additive masks become packed texts: a
 * query i of a text sees key j of the same text iff (!causal || j <= i) and
 * (window < 0 || |i - j| <= window). The softmax is computed in f32 for every
 * form; QK^T products and all accumulation are f32-exact on MFMA.
 * --------------------------------------------------------------------- */
typedef struct inl_attn_desc {
  int32_t n_texts;                 /* >= 0 */
  const int32_t* cu_seqlens_host;  /* [n_texts + 1], cu[0] == 0, nondecreasing */
  int32_t h_q;                     /* query heads */
  int32_t h_kv;                    /* key/value heads, h_q % h_kv == 0 */
  int32_t head_dim;                /* 8..256, multiple of 8 */
  int32_t causal;                  /* 0 or 1 */
  int32_t window;                  /* -1 = none, else inclusive radius >= 0 */
  float scale;                     /* multiplies q.k before the softmax */
  int32_t dtype;                   /* enum inl_dtype of q, k, v */
  int32_t out_dtype;               /* enum inl_dtype of out */
  int64_t q_row_stride;            /* elements between token rows; 0 = h_q*head_dim */
  int64_t k_row_stride;            /* 0 = h_kv*head_dim */
  int64_t v_row_stride;            /* 0 = h_kv*head_dim */
  int64_t o_row_stride;            /* 0 = h_q*head_dim */
  int32_t flags;                   /* INL_ATTN_* bits, 0 = defaults */
  /* Optional [n_texts]: the first row of text b in q, k, v and out (its
   * length stays cu_seqlens_host[b+1] - cu_seqlens_host[b]). NULL = packed,
   * text b starts at cu_seqlens_host[b]. With it a padded [B, T] batch runs
   * in place: start b*T + pad_b for the left padding of
   * crates/inl-core/src/attention.rs:126-199, b*T for the right padding of
   * gemma2.rs:499-523 and modernbert.rs:594-617. Rows outside every text are
   * not written (the reference leaves padded rows unspecified,
   * attention.rs:213-214). */
  const int32_t* seq_starts_host;
} inl_attn_desc;

/* bf16 inputs: the PV product runs in fp16 by default. V is converted to
 * fp16 while staged: exact for 2^-14 <= |v| < 65520 (bf16's 8 significant
 * bits fit fp16's 11); smaller values round to fp16 subnormals (absolute
 * error <= 2^-25); |v| >= 65520 becomes inf: the rows that see such a key
 * come out inf or NaN, and so may other rows of the same text (a masked
 * weight 0 times inf is NaN); other texts are unaffected. P is rounded to
 * fp16. Callers whose V is not normalised (Qwen3, ModernBERT, Qwen3.5: V
 * straight from the projection) and can reach 65520 set this flag, which
 * keeps V and P in bf16 (any range, 8x coarser P). */
#define INL_ATTN_PV_BF16 1

/* f32 descs: a batch too small to fill the GPU (fewer query blocks x head
 * groups than workgroups the GPU holds at once) has its longer query blocks'
 * key ranges split into parts that run as separate workgroups, and a second
 * kernel merges the parts' partial outputs (max, sum and unnormalised O,
 * kept in the plan's device memory). Results then differ from the unsplit
 * order of summation by f32 rounding only. This flag keeps every block in
 * one workgroup (one launch, no partials). bf16 descs are never split. */
#define INL_ATTN_NO_SPLIT 2

/* An attention plan: the packed texts' tile schedule, resident on the
 * device. Build it once per batch and reuse it for every layer of that
 * batch that has the same desc fields (all layers of one kind). */
typedef struct inl_attn_plan inl_attn_plan;

/* Build a plan (host work + one blocking upload). The desc's pointer fields
 * are read during the call only. The plan belongs to the device that is
 * current when it is created: its schedule lives there, and the kernel's
 * launch attributes are set there once, so inl_attn_fwd takes no lock. */
int inl_attn_plan_create(const inl_attn_desc* desc, inl_attn_plan** plan);
/* The same plan with its schedule in the caller's device `workspace` (at
 * least inl_attn_workspace_size() bytes, 16-byte aligned), uploaded
 * asynchronously on `stream` from the plan's own host copy of the schedule,
 * which lives until the plan is destroyed: nothing is allocated on the
 * device. The workspace must outlive the plan's launches; destroying the
 * plan does not free it. */
int inl_attn_plan_create_in(const inl_attn_desc* desc, void* workspace,
                            size_t workspace_bytes, void* stream,
                            inl_attn_plan** plan);
int inl_attn_plan_destroy(inl_attn_plan* plan);
/* Tiles the plan launches and query rows each covers (for reporting). */
int inl_attn_plan_info(const inl_attn_plan* plan, int64_t* n_tiles,
                       int32_t* block_m, int32_t* block_n);

/* out[N, h_q, head_dim] = attention(q[N, h_q, d], k[N, h_kv, d], v[N, h_kv, d]). */
int inl_attn_fwd(const inl_attn_plan* plan, const void* q, const void* k,
                 const void* v, void* out, void* stream);

/* One-shot form: plans into `workspace` (device memory of at least
 * inl_attn_workspace_size() bytes, 16-byte aligned) and launches. It
 * allocates no device or pinned memory: the schedule is built in host memory
 * and copied into the workspace with hipMemcpyAsync from pageable memory,
 * which orders behind the stream's earlier work. The workspace must stay
 * untouched until the launch has completed on `stream`. */
int inl_attn_workspace_size(const inl_attn_desc* desc, size_t* bytes);
int inl_attn_varlen_fwd(const inl_attn_desc* desc, const void* q,
                        const void* k, const void* v, void* out,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free one-shot form. It has no counterpart in the reference: it
 * is for callers that cannot allocate device memory per call (tight serving
 * loops, harnesses that forbid hipMalloc). It runs the same kernels as
 * inl_attn_varlen_fwd with INL_ATTN_NO_SPLIT set (the same results for
 * every bf16 desc; f32 batches are not split), but keeps the schedule in a
 * static device buffer of the library, INL_ATTN_STATIC_SCHEDULE_BYTES per
 * GPU (held by each GPU the library runs on until the process ends), so it
 * takes no workspace and calls no allocator. A batch whose schedule is
 * larger (about 200k units of work: far beyond any batch an engine plans)
 * fails with INL_E_INVALID. All calls on one GPU share that buffer: calls
 * in order on one stream are safe, while calls that overlap on one GPU (two
 * streams, or two host threads on different streams) race and must be
 * serialised by the caller. */
#define INL_ATTN_STATIC_SCHEDULE_BYTES (4u << 20)
int inl_attn_varlen_fwd_static(const inl_attn_desc* desc, const void* q,
                               const void* k, const void* v, void* out,
                               void* stream);

/* Host only: the name of the kernel a plan for `desc` launches (a static
 * string, e.g. "attn_pp_kernel<128, 64>"), for reporting and tests. The
 * bf16 fast kernels address each text's rows with 32-bit offsets; a text
 * whose q, k, v or out rows span 4 GiB or more takes the generic kernel. */
int inl_attn_kernel_name(const inl_attn_desc* desc, const char** name);

/* ------------------------------------------------------------------------
 * Prologue: fused per-head RMSNorm + RoPE over packed rows.
 *
 * Replaces q_norm/k_norm + rope of crates/inl-text/src/qwen3/mod.rs:236-249
 * (RmsNorm :72-90, RotaryTable :123-159), the q/k/v norms and rope of
 * gemma2.rs:389-410, rope_thd of modernbert.rs:264-269, the zero-centred
 * norms (weight = 1 + w, folded by the caller) and partial RoPE of
 * qwen3_5.rs:188-206,289-300, and the axial RoPE of vision.rs:792-800.
 *
 * y = rope(rms_norm(x) * weight) per (token, head) row of head_dim elements:
 *   norm:  x / sqrt(mean(x^2) + eps) * weight   (weight NULL = all ones;
 *          norm == 0 skips the norm);
 *   rope:  sections == 1: the first rotary_dim features are rotated in
 *          half-split pairs (i, i + rotary_dim/2) with cos/sin row
 *          rows[token] (the token's position inside its text; positions
 *          restart at 0 per packed text); the rest pass through.
 *          sections == 2 (axial): each half of the head is rotated by its
 *          own half-split, the first half with cos/sin, the second with
 *          cos2/sin2, tables indexed by rows[token] (per-token tables).
 *          rotary_dim == 0 skips the rope.
 * Tables are f32 `[table_rows, rotary_dim / 2]` (sections 1) or
 * `[table_rows, head_dim / 4]` (sections 2). A row index outside
 * [0, table_rows) yields NaN for that token instead of an out-of-range read.
 * round_tables = 1 rounds table values to bf16 (the reference stores tables
 * in the model dtype); round_norm = 1 rounds the normalised value to the
 * output dtype before the rotation (the reference materialises it).
 * In-place operation (y == x, same strides) is allowed.
 * --------------------------------------------------------------------- */
typedef struct inl_norm_rope_desc {
  int64_t n_tokens;
  int32_t heads;
  int32_t head_dim;               /* multiple of 8, <= 512 */
  int64_t x_row_stride;           /* elements; 0 = heads*head_dim */
  int64_t y_row_stride;           /* elements; 0 = heads*head_dim */
  int32_t dtype;                  /* x dtype */
  int32_t out_dtype;              /* y dtype */
  int32_t norm;                   /* 1 = apply the RMSNorm */
  float eps;
  int32_t rotary_dim;             /* 0 = no rope; sections 1: 8 or a multiple of 16 <= head_dim */
  int32_t sections;               /* 1 = half-split, 2 = axial */
  int32_t table_rows;
  int32_t round_tables;
  int32_t round_norm;
} inl_norm_rope_desc;

int inl_norm_rope_fwd(const inl_norm_rope_desc* desc, const void* x, void* y,
                      const void* weight /* [head_dim], dtype, or NULL */,
                      const int32_t* rows /* [n_tokens] device, table row per token */,
                      const float* cos, const float* sin,
                      const float* cos2, const float* sin2, void* stream);

/* The q and k heads of one row in one launch: heads [0, q_heads) of each
 * row are normalised with q_weight, heads [q_heads, desc->heads) with
 * k_weight (NULL = all ones), every head rotated as inl_norm_rope_fwd does.
 * For the q and k slices of a fused projection row (q heads then k heads,
 * x_row_stride the fused row), the two per-tensor calls of the reference's
 * attention prologue (qwen3/mod.rs:236-249: q_norm, k_norm, then rope of q
 * and of k) become one launch over the same bytes. 0 < q_heads <
 * desc->heads. Results equal two inl_norm_rope_fwd calls, bit for bit. */
int inl_norm_rope_qk_fwd(const inl_norm_rope_desc* desc, int32_t q_heads,
                         const void* x, void* y, const void* q_weight,
                         const void* k_weight, const int32_t* rows,
                         const float* cos, const float* sin,
                         const float* cos2, const float* sin2, void* stream);

/* Host helper: text-local positions of packed tokens (0..len-1 per text),
 * written to a host array of cu_seqlens_host[n_texts] entries. */
int inl_positions_host(int32_t n_texts, const int32_t* cu_seqlens_host, int32_t* positions);

/* Host helper: RoPE tables as the reference builds them.
 * mode 0: inv_freq and angles in f64, stored f32 (qwen3/mod.rs:131-153,
 *         gemma2.rs:292-315, modernbert.rs:239-262);
 * mode 1: in f32 (qwen3_5.rs:940-957). cos/sin are host [positions, dim/2]. */
int inl_rope_table_host(int32_t rotary_dim, double theta, int32_t positions,
                        int32_t mode, float* cos_out, float* sin_out);

/* ------------------------------------------------------------------------
 * Epilogues. `cu` is a DEVICE int32 array [n_texts + 1] of packed row
 * offsets (cu[0] == 0, nondecreasing); outputs are f32.
 * --------------------------------------------------------------------- */

/* Last-token pooling: pooled[b] = l2(rms_norm(hidden[cu[b+1]-1]) * weight),
 * [n_texts, hidden_dim]. Replaces the final norm of the last position and
 * the L2 normalisation of crates/inl-text/src/qwen3/mod.rs:356-357, 464-469
 * (l2: x / sqrt(sum x^2 + 1e-12)). round_norm = 1 rounds the normed row to
 * bf16 before the L2 (the reference keeps it in the model dtype). Empty
 * texts yield zero rows. weight NULL = all ones. */
int inl_pool_last_fwd(int32_t n_texts, const int32_t* cu, int32_t hidden_dim,
                      int64_t row_stride, int32_t dtype, const void* hidden,
                      const void* weight, float eps, int32_t round_norm,
                      float* pooled, void* stream);

/* Mean pooling: pooled[b] = sum of the rows of text b / len_b,
 * [n_texts, hidden_dim] (crates/inl-text/src/gemma2.rs:647-656); empty texts
 * give zeros. normalize = 1 also L2-normalises each row with 1e-12 inside
 * the square root (gemma2.rs:660-661, for an identity projection). */
int inl_pool_mean_fwd(int32_t n_texts, const int32_t* cu, int32_t hidden_dim,
                      int64_t row_stride, int32_t dtype, const void* hidden,
                      int32_t normalize, float* pooled, void* stream);

/* Row-wise L2 normalisation of the first `dim` entries of f32 rows (in place
 * allowed): x / sqrt(sum x^2 + eps_inside). eps_inside = 1e-12 is the
 * pooled-embedding norm (qwen3/mod.rs:468); eps_inside = 0 with
 * skip_zero = 1 is the Matryoshka truncate-and-renormalise of
 * crates/inl-text/src/native.rs:822-830 (rows of norm 0 are left as is). */
int inl_l2_normalize_fwd(int32_t rows, int32_t dim, int64_t in_stride,
                         const float* x, int64_t out_stride, float* y,
                         float eps_inside, int32_t skip_zero, void* stream);

/* SPLADE pooling (crates/inl-sparse/src/modernbert.rs:806-907):
 *   m[r, t]   = max over speaking positions p in [offs[r], offs[r+1]) of
 *               logits[p, t]  (f32, bias-free; -inf if the row has none);
 *   w[r, t]   = ln(relu(m + bias[t] - shift) * open[t] + 1), open[t] = 0 for
 *               the masked vocabulary ids (at most 16);
 *   out[r, c] = max(0, max over t with canonical[t] == c of w[r, t])
 *               (canonical NULL: out = w and out_dim == vocab).
 * offs: DEVICE int32 [rows + 1]. bias NULL = no bias. out: [rows, out_dim].
 * canonical: DEVICE int32 [vocab] with 0 <= canonical[t] < out_dim; an id
 * outside that range is skipped (its term is dropped, nothing is written). 
 * The max and the fold do not depend on evaluation order: for given logits
 * the output, and its active-term set {c : out > 0}, is bit-exact. */
int inl_pool_splade_fwd(int32_t rows, const int32_t* offs, int32_t vocab,
                        const float* logits, int64_t logits_stride,
                        const float* bias, float shift,
                        const int32_t* masked_ids_host, int32_t n_masked,
                        const int32_t* canonical, int32_t out_dim, float* out,
                        void* stream);

/* The finish and fold of inl_pool_splade_fwd applied to per-row maxima that
 * are already known (`maxima` [rows, vocab] f32, -inf for a silent row, e.g.
 * from inl_splade_decoder_max_fwd): out[r, c] = max(0, max over t with
 * canonical[t] == c of ln(relu(maxima[r, t] + bias[t] - shift) * open[t] + 1))
 * (crates/inl-sparse/src/modernbert.rs:874-907). */
int inl_splade_finish_fwd(int32_t rows, int32_t vocab, const float* maxima,
                          int64_t maxima_stride, const float* bias, float shift,
                          const int32_t* masked_ids_host, int32_t n_masked,
                          const int32_t* canonical, int32_t out_dim, float* out,
                          void* stream);

/* ------------------------------------------------------------------------ */
/* Packed batch planner (host). Replaces the padded planners of the text,
 * sparse, late and vision engines (crates/inl-text/src/native.rs:698-735,
 * crates/inl-sparse/src/native.rs:557-582, crates/inl-late/src/native.rs:
 * 694-719, crates/inl-vision/src/engine.rs:782-798), which split inputs in
 * order into consecutive batches of at most `batch_size` inputs and at most
 * `max_batch_tokens` PADDED tokens (inputs x longest), plus, for text, an
 * attention-score budget. Packed into one cu_seqlens row set, a batch costs
 * its REAL tokens: this planner caps sum(lengths) instead, and the fused
 * attention keeps no score matrix, so no score budget applies.
 *   lengths:   host [n] token counts, in the caller's order (>= 0; a length of
 *              0 counts as 1 token, as the reference's `length.max(1)`);
 *   batch_end: host [n], receives each batch's exclusive end index;
 *   n_batches: receives the number of batches (0 for n == 0).
 * A single input over `max_tokens` forms a batch by itself, as in the
 * reference. The split is greedy, and greedy is optimal here (fewest
 * batches) because a feasible batch stays feasible without its first input. */
int inl_plan_packed_batches(const int32_t* lengths, int64_t n, int64_t max_items, int64_t max_tokens,
                            int64_t* batch_end, int64_t* n_batches);

/* ------------------------------------------------------------------------ */
const char* inl_last_error(void);
int32_t inl_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* INL_HIP_H */
