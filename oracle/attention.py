"""Attention oracle (numpy). TEST INFRASTRUCTURE ONLY - never on the product path.

Two families of functions live here:

1. Restatements of the reference's *padded* attention forms, one per model,
   with the reference's additive masks (values, dtypes and the way they are
   summed) and its scale conventions. Tensors are ``[batch, heads, seq, dim]``.
2. ``varlen_attention``: the *packed* variable-length form the HIP kernels
   implement - texts back to back in ``[tokens, heads, dim]`` rows, a query
   attends only to keys of its own text within the form's mask. Tests pin it
   to (1) on the real rows of every form (packing invariance), to a brute
   force softmax, and to the reference's own invariants.

All arithmetic is float64 unless ``dtype=np.float32`` is passed.
"""
from __future__ import annotations

import numpy as np

# attention.rs:28 (Qwen3), qwen3_5.rs:16 (Qwen3.5), modernbert.rs:595 (ModernBERT)
MASK_VALUE_1E4 = -1e4
# gemma2.rs:40 (EmbeddingGemma 2), vision.rs:29 (vision tower)
MASK_VALUE_1E9 = -1e9
# attention.rs:25, modernbert.rs:214, qwen3_5.rs:19, vision.rs:35
QUERY_TILE = 256


# ---------------------------------------------------------------------------
# Deterministic inputs the reference's own unit tests use.
# ---------------------------------------------------------------------------

def pseudo(n: int, seed: int, offset: int = 1) -> np.ndarray:
    """Values in [-0.5, 0.5) from the reference tests' LCG.

    ``offset=1`` is ``pseudo`` in crates/inl-core/src/attention.rs:327-336;
    ``offset=7`` is the variant in crates/inl-text/src/qwen3/mod.rs:488-496
    (same LCG, different start). u32 wrapping arithmetic, f32 result.
    """
    state = (seed * 2_654_435_761 + offset) & 0xFFFFFFFF
    out = np.empty(n, dtype=np.float32)
    for i in range(n):
        state = (state * 1_664_525 + 1_013_904_223) & 0xFFFFFFFF
        out[i] = np.float32(state >> 8) / np.float32(1 << 24) - np.float32(0.5)
    return out


# ---------------------------------------------------------------------------
# Shared pieces
# ---------------------------------------------------------------------------

def repeat_kv(x: np.ndarray, n_rep: int) -> np.ndarray:
    """``[B, Nkv, T, D] -> [B, Nkv*n_rep, T, D]``; query head h reads KV head
    h // n_rep (crates/inl-core/src/attention.rs:202-210; the Gemma2 and
    vision ``repeat`` closures, gemma2.rs:421-429, vision.rs:320-327)."""
    if n_rep == 1:
        return x
    b, kv, t, d = x.shape
    return np.broadcast_to(x[:, :, None], (b, kv, n_rep, t, d)).reshape(b, kv * n_rep, t, d)


def softmax_last(x: np.ndarray) -> np.ndarray:
    """Numerically stable softmax over the last axis (candle
    ``softmax_last_dim`` / ``ops::softmax``)."""
    m = np.max(x, axis=-1, keepdims=True)
    e = np.exp(x - m)
    return e / np.sum(e, axis=-1, keepdims=True)


# ---------------------------------------------------------------------------
# Qwen3 (crates/inl-core/src/attention.rs)
# ---------------------------------------------------------------------------

def qwen3_additive_mask(pad_lens, seq: int, dtype=np.float64) -> np.ndarray:
    """``[B, 1, T, T]``: MASK_VALUE for ``key > query`` plus MASK_VALUE for
    ``key < pad`` - summed, so -2e4 where both hold
    (attention.rs:170-199, pinned by its test at :404-432)."""
    pos = np.arange(seq)
    future = (pos[None, :] > pos[:, None]).astype(dtype) * MASK_VALUE_1E4
    pads = np.asarray(pad_lens).reshape(-1, 1, 1)
    padding = (pos.reshape(1, 1, seq) < pads).astype(dtype) * MASK_VALUE_1E4
    return (future[None] + padding)[:, None].astype(dtype)


def qwen3_eager(q, k, v, mask, scale, n_rep):
    """attention.rs:236-249: scores = q k^T * scale + mask; softmax; @ v."""
    k = repeat_kv(k, n_rep)
    v = repeat_kv(v, n_rep)
    scores = (q @ np.swapaxes(k, 2, 3)) * scale
    return softmax_last(scores + mask) @ v


def qwen3_tiled(q, k, v, mask, scale, n_rep, tile=QUERY_TILE):
    """attention.rs:251-278: q is scaled first, then query tiles of ``tile``
    rows each take matmul, mask add, softmax and matmul."""
    seq = q.shape[2]
    k = repeat_kv(k, n_rep)
    v = repeat_kv(v, n_rep)
    kt = np.swapaxes(k, 2, 3)
    q = q * scale
    blocks = []
    for start in range(0, seq, tile):
        rows = min(tile, seq - start)
        s = q[:, :, start:start + rows] @ kt + mask[:, :, start:start + rows]
        blocks.append(softmax_last(s) @ v)
    return np.concatenate(blocks, axis=2)


def flash_attention_1(q, k, v, scale, causal, block=16, dtype=np.float64):
    """Online-softmax attention for one text: ``q [T, H, D]``, ``k, v [T, H, D]``
    (heads already matched). Keys are visited in blocks of ``block`` with a
    running max and sum, the algorithm of candle's CPU ``flash_attn`` that
    attention.rs:282-315 calls per unpadded row."""
    t, h, d = q.shape
    qf = q.astype(dtype)
    kf = k.astype(dtype)
    vf = v.astype(dtype)
    out = np.zeros((t, h, d), dtype=dtype)
    for head in range(h):
        m = np.full(t, -np.inf, dtype=dtype)
        l = np.zeros(t, dtype=dtype)
        acc = np.zeros((t, d), dtype=dtype)
        for j0 in range(0, t, block):
            j1 = min(t, j0 + block)
            s = (qf[:, head] @ kf[j0:j1, head].T) * dtype(scale)
            if causal:
                qi = np.arange(t)[:, None]
                kj = np.arange(j0, j1)[None, :]
                s = np.where(kj <= qi, s, -np.inf)
            m_new = np.maximum(m, s.max(axis=1))
            base = np.where(np.isneginf(m_new), 0.0, m_new).astype(dtype)
            p = np.exp(s - base[:, None])
            alpha = np.exp(np.where(np.isneginf(m), -np.inf, m - base))
            l = l * alpha + p.sum(axis=1)
            acc = acc * alpha[:, None] + p @ vf[j0:j1, head]
            m = m_new
        out[:, head] = acc / l[:, None]
    return out


def qwen3_cpu_flash(q, k, v, pad_lens, scale, dtype=np.float64):
    """attention.rs:282-315: per batch row, flash attention on the real
    (unpadded) tokens with a causal mask; padding rows are zero. GQA is
    handled by matching KV heads (candle's flash_attn broadcasts them)."""
    b, h, seq, d = q.shape
    n_rep = h // k.shape[1]
    out = np.zeros((b, h, seq, d), dtype=dtype)
    for row, pad in enumerate(pad_lens):
        take = lambda t: np.swapaxes(t[row, :, pad:], 0, 1)  # [T, H, D]
        kk = repeat_kv(k[row:row + 1], n_rep)[0]
        vv = repeat_kv(v[row:row + 1], n_rep)[0]
        o = flash_attention_1(take(q), np.swapaxes(kk[:, pad:], 0, 1),
                              np.swapaxes(vv[:, pad:], 0, 1), scale, True, dtype=dtype)
        out[row, :, pad:] = np.swapaxes(o, 0, 1)
    return out


# ---------------------------------------------------------------------------
# EmbeddingGemma 2 text (crates/inl-text/src/gemma2.rs)
# ---------------------------------------------------------------------------

def gemma2_attention_mask(lens, seq: int, window):
    """gemma2.rs:499-523: ``[B, 1, T, T]`` f32, -1e9 where ``key >= len`` or
    (sliding) ``|q - k| > window``; ``None`` when nothing is masked."""
    padded = any(l < seq for l in lens)
    windowed = window is not None and window + 1 < seq
    if not padded and not windowed:
        return None
    pos = np.arange(seq)
    out = np.zeros((len(lens), 1, seq, seq), dtype=np.float32)
    for row, ln in enumerate(lens):
        blocked = pos[None, :] >= ln
        if window is not None:
            blocked = blocked | (np.abs(pos[:, None] - pos[None, :]) > window)
        out[row, 0][np.broadcast_to(blocked, (seq, seq))] = MASK_VALUE_1E9
    return out


def gemma2_attention(q, k, v, mask):
    """gemma2.rs:414-441: repeat KV, scores = q k^T (scale 1, q/k are RMS
    normalised), upcast to f32, + mask, softmax, downcast, @ v."""
    groups = q.shape[1] // k.shape[1]
    k = repeat_kv(k, groups)
    v = repeat_kv(v, groups)
    s = q @ np.swapaxes(k, 2, 3)
    if mask is not None:
        s = s + mask
    return softmax_last(s) @ v


# ---------------------------------------------------------------------------
# ModernBERT (crates/inl-sparse/src/modernbert.rs)
# ---------------------------------------------------------------------------

def modernbert_masks(lengths, seq: int, half_window: int, dtype=np.float64):
    """modernbert.rs:594-617: (global, local) ``[B, 1, T, T]``; -1e4 on
    padding keys in both; local also masks ``|k - q| > half_window``
    (``half_window = local_attention / 2``, modernbert.rs:543)."""
    pos = np.arange(seq)
    b = len(lengths)
    glob = np.zeros((b, 1, seq, seq), dtype=dtype)
    loc = np.zeros((b, 1, seq, seq), dtype=dtype)
    far = np.abs(pos[None, :] - pos[:, None]) > half_window
    for row, ln in enumerate(lengths):
        pad = np.broadcast_to(pos[None, :] >= ln, (seq, seq))
        glob[row, 0][pad] = MASK_VALUE_1E4
        loc[row, 0][pad | far] = MASK_VALUE_1E4
    return glob, loc


def modernbert_attend(q, k, v, mask, scale, tile=QUERY_TILE):
    """modernbert.rs:366-401 (tiled backend): q * scale, query tiles,
    + mask, softmax, @ v. MHA (no GQA)."""
    return qwen3_tiled(q, k, v, mask, scale, 1, tile)


# ---------------------------------------------------------------------------
# Qwen3.5 full attention (crates/inl-late/src/qwen3_5.rs)
# ---------------------------------------------------------------------------

def qwen35_mask(lengths, t: int, causal: bool, dtype=np.float64):
    """qwen3_5.rs:914-934: -1e4 on keys past each row's length, plus -1e4 on
    the future when causal (summed). ``[B,1,1,T]`` or ``[B,1,T,T]``."""
    keys = np.arange(t).reshape(1, 1, 1, t)
    limits = np.asarray(lengths).reshape(-1, 1, 1, 1)
    padding = (keys >= limits).astype(dtype) * MASK_VALUE_1E4
    if not causal:
        return padding
    queries = np.arange(t).reshape(1, 1, t, 1)
    future = (keys > queries).astype(dtype) * MASK_VALUE_1E4
    return future + padding


def qwen35_grouped_tiled(q, k, v, mask, scale, n_rep, tile=QUERY_TILE):
    """qwen3_5.rs:364-407: query groups folded into GEMM rows (equal to
    repeat_kv), q * scale, + mask rows (the whole key mask when it is
    ``[B,1,1,T]``), softmax, @ v."""
    b, heads, t, d = q.shape
    kv = k.shape[1]
    q = q * scale
    kt = np.swapaxes(k, 2, 3)
    causal = mask is not None and mask.shape[2] > 1
    blocks = []
    for start in range(0, t, tile):
        rows = min(tile, t - start)
        query = q[:, :, start:start + rows].reshape(b, kv, n_rep * rows, d)
        s = (query @ kt).reshape(b, heads, rows, t)
        if mask is not None:
            s = s + (mask[:, :, start:start + rows] if causal else mask)
        w = softmax_last(s).reshape(b, kv, n_rep * rows, t)
        blocks.append((w @ v).reshape(b, heads, rows, d))
    return np.concatenate(blocks, axis=2)


# ---------------------------------------------------------------------------
# Vision tower (crates/inl-vision/src/vision.rs)
# ---------------------------------------------------------------------------

def vision_key_mask(padding):
    """vision.rs:567-574: ``[B, 1, 1, T]`` -1e9 on padding keys
    (``padding`` is a ``[B, T]`` 0/1 array, 1 = padding)."""
    p = np.asarray(padding, dtype=np.float64)
    return (p * MASK_VALUE_1E9).reshape(p.shape[0], 1, 1, p.shape[1])


def vision_masked_attention(q, k, v, mask, tile=QUERY_TILE):
    """vision.rs:226-259 (tiled): scale 1.0, + key mask, softmax, @ v."""
    seq = q.shape[2]
    kt = np.swapaxes(k, 2, 3)
    blocks = []
    for start in range(0, seq, tile):
        rows = min(tile, seq - start)
        s = q[:, :, start:start + rows] @ kt + mask
        blocks.append(softmax_last(s) @ v)
    return np.concatenate(blocks, axis=2)


# ---------------------------------------------------------------------------
# The packed variable-length form (what the HIP kernels compute)
# ---------------------------------------------------------------------------

def allowed(tq: int, tk: int, causal: bool, window: int) -> np.ndarray:
    """``[tq, tk]`` boolean: key j visible from query i of the same text.
    Causal: ``j <= i`` (attention.rs:184-186). Window: ``|i - j| <= window``,
    an inclusive radius (gemma2.rs:515, modernbert.rs:607,
    crates/inl-ane/src/layout.rs:400-403). ``window < 0`` = no window."""
    i = np.arange(tq)[:, None]
    j = np.arange(tk)[None, :]
    ok = np.ones((tq, tk), dtype=bool)
    if causal:
        ok &= j <= i
    if window is not None and window >= 0:
        ok &= np.abs(i - j) <= window
    return ok


def varlen_attention(q, k, v, cu_seqlens, *, causal: bool, window: int = -1,
                     scale: float = 1.0, dtype=np.float64) -> np.ndarray:
    """Packed attention: ``q [N, Hq, D]``, ``k, v [N, Hkv, D]``, texts at
    ``cu_seqlens[b]:cu_seqlens[b+1]``; query head h reads KV head
    ``h // (Hq // Hkv)``. Masked keys are excluded, which equals the
    reference's finite additive masks wherever a row has a visible key (every
    row does: j = i is always visible) - see the packing-invariance tests.
    Packed-segment semantics follow crates/inl-ane/src/layout.rs:1-7,391-415.
    Returns ``[N, Hq, D]`` in ``dtype``."""
    n, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = np.zeros((n, hq, d), dtype=dtype)
    qf, kf, vf = (x.astype(dtype) for x in (q, k, v))
    for b in range(len(cu_seqlens) - 1):
        s0, s1 = int(cu_seqlens[b]), int(cu_seqlens[b + 1])
        t = s1 - s0
        if t == 0:
            continue
        ok = allowed(t, t, causal, window)
        for h in range(hq):
            kh = h // g
            s = (qf[s0:s1, h] @ kf[s0:s1, kh].T) * dtype(scale)
            s = np.where(ok, s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            p = np.exp(s - m)
            out[s0:s1, h] = (p / p.sum(axis=1, keepdims=True)) @ vf[s0:s1, kh]
    return out


def pack(padded: np.ndarray, lengths, left_pad: bool) -> np.ndarray:
    """``[B, H, T, D]`` padded -> ``[N, H, D]`` packed real rows."""
    rows = []
    seq = padded.shape[2]
    for b, ln in enumerate(lengths):
        sl = slice(seq - ln, seq) if left_pad else slice(0, ln)
        rows.append(np.swapaxes(padded[b, :, sl], 0, 1))
    return np.concatenate(rows, axis=0)


def cu_from_lengths(lengths) -> np.ndarray:
    return np.concatenate([[0], np.cumsum(np.asarray(lengths, dtype=np.int64))]).astype(np.int32)


# ---------------------------------------------------------------------------
# Algorithmic work (what ``roofline.achieved`` counts)
# ---------------------------------------------------------------------------

def visible_pairs(lengths, causal: bool, window: int = -1) -> int:
    """Number of (query, key) pairs a packed call attends, summed over texts:
    causal ``T(T+1)/2``; full ``T^2``; window radius W
    ``sum_q min(T, q+W+1) - max(0, q-W)`` (with causal, ``min(q+1, ...)``)."""
    total = 0
    for t in lengths:
        t = int(t)
        if t <= 0:
            continue
        q = np.arange(t, dtype=np.int64)
        hi = np.full(t, t, dtype=np.int64) if not causal else q + 1
        lo = np.zeros(t, dtype=np.int64)
        if window is not None and window >= 0:
            hi = np.minimum(hi, q + window + 1)
            lo = np.maximum(lo, q - window)
        total += int(np.sum(hi - lo))
    return total


def attention_flops(lengths, h_q: int, head_dim: int, causal: bool, window: int = -1) -> int:
    """``4 * H_q * d * visible_pairs`` (QK^T and PV, 2 flops per MAC)."""
    return 4 * h_q * head_dim * visible_pairs(lengths, causal, window)
