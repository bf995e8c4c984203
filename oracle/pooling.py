"""Epilogue oracle: last-token, mean and SPLADE pooling (numpy).
TEST INFRASTRUCTURE ONLY - never on the product path.
"""
from __future__ import annotations

import numpy as np

from .prologue import rms_norm


def l2_normalize(x: np.ndarray, dtype=np.float64) -> np.ndarray:
    """``x / sqrt(sum(x^2) + 1e-12)`` per row, in f32 in the reference
    (crates/inl-text/src/qwen3/mod.rs:464-469, gemma2.rs:660-661)."""
    xf = x.astype(dtype)
    return xf / np.sqrt(np.sum(xf * xf, axis=-1, keepdims=True) + dtype(1e-12))


def last_token(hidden, cu_seqlens, norm_weight, eps, dtype=np.float64):
    """qwen3/mod.rs:339-358 + :464-469: final RMSNorm of each text's last
    row, then L2 normalisation. ``hidden [N, h]`` packed; returns ``[B, h]``.
    Packed equivalent of the left-padded last position (the last row of a
    segment; crates/inl-ane/src/layout.rs:444-451)."""
    cu = np.asarray(cu_seqlens)
    rows = hidden[cu[1:] - 1]
    return l2_normalize(rms_norm(rows, norm_weight, eps, dtype), dtype)


def mean_pool(hidden, cu_seqlens, dtype=np.float64):
    """gemma2.rs:647-656: ``sum_{t < len} h_t / len`` per text (the reference
    writes it as a ``[B,1,T] x [B,T,h]`` matmul with weight ``1/max(len,1)``).
    A zero-length text pools to zeros."""
    cu = np.asarray(cu_seqlens)
    out = np.zeros((len(cu) - 1, hidden.shape[1]), dtype=dtype)
    for b in range(len(cu) - 1):
        n = cu[b + 1] - cu[b]
        if n > 0:
            out[b] = hidden[cu[b]:cu[b + 1]].astype(dtype).sum(axis=0) / dtype(max(n, 1))
    return out


def truncate_and_normalize(vector: np.ndarray, dim: int) -> np.ndarray:
    """crates/inl-text/src/native.rs:822-830 (Matryoshka): keep the first
    ``dim`` entries, divide by their f32 norm when it is positive."""
    v = np.asarray(vector, dtype=np.float32)[..., :dim].copy()
    norm = np.sqrt(np.sum(v * v, axis=-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    return np.where(norm > 0, v / np.where(norm > 0, norm, 1), v).astype(np.float32)


# ---------------------------------------------------------------------------
# SPLADE (crates/inl-sparse/src/modernbert.rs:695-907)
# ---------------------------------------------------------------------------

def speakers(rows, prefix_token_ids, seq=None):
    """modernbert.rs:703-716: packed speaking positions (real, non-prefix
    tokens), row by row. Returns (index into the packed token rows, ends)."""
    index, ends, base = [], [], 0
    prefix = set(int(p) for p in prefix_token_ids)
    for ids in rows:
        for pos, tok in enumerate(ids):
            if int(tok) not in prefix:
                index.append(base + pos)
        ends.append(len(index))
        base += len(ids) if seq is None else seq
    return np.asarray(index, dtype=np.int64), np.asarray(ends, dtype=np.int64)


def splade_row_max(logits: np.ndarray, ends) -> np.ndarray:
    """Per-row running max over the speaking positions of the bias-free
    logits (modernbert.rs:837-863); ``-inf`` for a row with none
    (:864-871). ``logits [n_speak, V]`` f32, exact in any order."""
    ends = np.asarray(ends)
    out = np.full((len(ends), logits.shape[1]), -np.inf, dtype=np.float32)
    begin = 0
    for r, end in enumerate(ends):
        if end > begin:
            out[r] = logits[begin:end].max(axis=0)
        begin = end
    return out


def splade_finish(pooled, bias, shift: float, masked_vocab_ids) -> np.ndarray:
    """modernbert.rs:879-885 in f32: ``ln(relu(max + bias - shift) * open + 1)``
    with ``open`` 0 on masked vocabulary ids; relu runs before the mask so
    ``-inf`` never meets a zero."""
    logit = pooled.astype(np.float32)
    if bias is not None:
        logit = (logit + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    x = (logit - np.float32(shift)).astype(np.float32)
    x = np.maximum(x, np.float32(0.0))
    open_ = np.ones(pooled.shape[1], dtype=np.float32)
    open_[np.asarray(masked_vocab_ids, dtype=np.int64)] = 0.0
    x = (x * open_[None, :]).astype(np.float32)
    return np.log((x + np.float32(1.0)).astype(np.float32)).astype(np.float32)


def splade_fold(weights: np.ndarray, canonical_ids) -> np.ndarray:
    """modernbert.rs:888-907: max-fold the vocabulary onto canonical terms;
    the output starts at 0 and a slot takes a weight only if it is larger."""
    if canonical_ids is None:
        return weights
    canon = np.asarray(canonical_ids, dtype=np.int64)
    width = int(canon.max()) + 1
    out = np.zeros((weights.shape[0], width), dtype=np.float32)
    for r in range(weights.shape[0]):
        np.maximum.at(out[r], canon, weights[r])
    return out


def splade_pool(logits, ends, bias, shift, masked_vocab_ids, canonical_ids):
    """The whole SPLADE epilogue: row max, finish, fold."""
    return splade_fold(splade_finish(splade_row_max(logits, ends), bias, shift,
                                     masked_vocab_ids), canonical_ids)


def sparse_from_pairs(dense_row):
    """crates/inl-sparse/src/lib.rs:51-62: keep finite, positive weights,
    sorted by index. Returns (indices u32, values f32)."""
    w = np.asarray(dense_row, dtype=np.float32)
    keep = np.isfinite(w) & (w > 0)
    idx = np.nonzero(keep)[0].astype(np.uint32)
    return idx, w[keep]
