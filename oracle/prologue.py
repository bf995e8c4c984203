"""Prologue oracle: per-head RMSNorm and rotary embeddings (numpy).
TEST INFRASTRUCTURE ONLY - never on the product path.

The reference applies, per attention layer, a per-head RMSNorm to q and k
(and a weightless one to v for EmbeddingGemma and the vision tower), then a
half-split RoPE. The HIP prologue kernel fuses both over packed rows whose
positions restart at 0 for every text.
"""
from __future__ import annotations

import numpy as np


def rms_norm(x: np.ndarray, weight, eps: float, dtype=np.float64) -> np.ndarray:
    """``x / sqrt(mean(x^2) + eps) * w`` over the last axis: candle
    ``ops::rms_norm`` as called by crates/inl-text/src/qwen3/mod.rs:86-90 and
    pinned to this textbook form by its test at :706-730. ``weight=None`` is
    the weightless (all-ones) norm of gemma2.rs:409-410 / vision.rs v_norm."""
    xf = x.astype(dtype)
    ms = np.mean(xf * xf, axis=-1, keepdims=True)
    y = xf / np.sqrt(ms + dtype(eps))
    if weight is not None:
        y = y * np.asarray(weight, dtype=dtype)
    return y


def rope_table(rotary_dim: int, theta: float, positions: int):
    """``cos, sin [positions, rotary_dim/2]``: inv_freq and angles computed in
    f64, stored as f32 (crates/inl-text/src/qwen3/mod.rs:131-153; the same
    construction at gemma2.rs:292-315 and modernbert.rs:239-262)."""
    half = rotary_dim // 2
    inv = 1.0 / np.power(float(theta), (2.0 * np.arange(half)) / rotary_dim)
    ang = np.arange(positions, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rope_table_f32(rotary_dim: int, theta: float, positions: int):
    """Qwen3.5's table (crates/inl-late/src/qwen3_5.rs:940-957): inv_freq
    ``1 / theta^(2i/dim)`` and the angle products in f32."""
    half = rotary_dim // 2
    th = np.float32(theta)
    inv = np.array([np.float32(1.0) / np.power(th, np.float32(2 * i) / np.float32(rotary_dim))
                    for i in range(half)], dtype=np.float32)
    steps = np.arange(positions, dtype=np.float32)[:, None]
    f = (steps * inv[None, :]).astype(np.float32)
    return np.cos(f).astype(np.float32), np.sin(f).astype(np.float32)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Half-split rotation of the last axis: pairs ``(x[i], x[i + d/2])``
    rotated by the angle of column i. ``cos``/``sin`` broadcast against
    ``x[..., :d/2]``. This is candle ``rotary_emb::rope`` / ``rope_thd``
    (qwen3/mod.rs:120-127,248-249), pinned by the reference to
    ``x * [cos, cos] + rotate_half(x) * [sin, sin]`` (qwen3/mod.rs:162-179,
    test :678-703)."""
    half = x.shape[-1] // 2
    x1 = x[..., :half]
    x2 = x[..., half:]
    return np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1)


def rope_manual(x, cos, sin):
    """The reference's test spelling: ``x*[cos,cos] + rotate_half(x)*[sin,sin]``
    with ``rotate_half(x) = [-x2, x1]`` (qwen3/mod.rs:162-179)."""
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * np.concatenate([cos, cos], -1) + rot * np.concatenate([sin, sin], -1)


def partial_rope(x, cos, sin, rotary_dim: int):
    """qwen3_5.rs:289-300: rotate the first ``rotary_dim`` features, pass the
    rest through."""
    if rotary_dim == x.shape[-1]:
        return rope(x, cos, sin)
    return np.concatenate([rope(x[..., :rotary_dim], cos, sin), x[..., rotary_dim:]], axis=-1)


def vision_inv_freq(head_dim: int, theta: float) -> np.ndarray:
    """vision.rs:760-767: ``spatial = head_dim/2``; inv_freq over
    ``spatial/2`` entries, computed in f32."""
    spatial = head_dim // 2
    th = np.float32(theta)
    return np.array([np.float32(1.0) / np.power(th, np.float32(2 * i) / np.float32(spatial))
                     for i in range(spatial // 2)], dtype=np.float32)


def axial_tables(inv_freq: np.ndarray, pos_xy: np.ndarray):
    """vision.rs:771-780: per-token tables ``[tokens, head_dim/4]`` from
    ``pos_xy [tokens, 2]`` (f32): (cos_x, sin_x, cos_y, sin_y)."""
    px = pos_xy[:, 0:1].astype(np.float32) * inv_freq[None, :]
    py = pos_xy[:, 1:2].astype(np.float32) * inv_freq[None, :]
    return (np.cos(px).astype(np.float32), np.sin(px).astype(np.float32),
            np.cos(py).astype(np.float32), np.sin(py).astype(np.float32))


def axial_rope(x, cx, sx, cy, sy):
    """vision.rs:792-800: the head splits into an x-half and a y-half, each
    rotated by its own half-split RoPE. ``x [tokens, heads, D]``, tables
    ``[tokens, D/4]``."""
    half = x.shape[-1] // 2
    lo = rope(x[..., :half], cx[:, None, :], sx[:, None, :])
    hi = rope(x[..., half:], cy[:, None, :], sy[:, None, :])
    return np.concatenate([lo, hi], axis=-1)


def positions_of(cu_seqlens) -> np.ndarray:
    """Packed rows' positions: 0.. within each text (positions restart per
    segment, crates/inl-ane/src/layout.rs:5-7)."""
    cu = np.asarray(cu_seqlens)
    n = int(cu[-1])
    pos = np.empty(n, dtype=np.int64)
    for b in range(len(cu) - 1):
        pos[cu[b]:cu[b + 1]] = np.arange(cu[b + 1] - cu[b])
    return pos


def norm_rope_packed(x, cu_seqlens, weight, eps, cos, sin, rotary_dim=None,
                     norm=True, rope_on=True, dtype=np.float64):
    """The fused prologue over packed rows ``x [N, H, D]``: optional RMSNorm
    (``weight=None`` = weightless), then RoPE on the first ``rotary_dim``
    features at each row's text-local position."""
    y = rms_norm(x, weight, eps, dtype) if norm else x.astype(dtype)
    if not rope_on:
        return y
    rd = rotary_dim or x.shape[-1]
    pos = positions_of(cu_seqlens)
    c = cos[pos][:, None, :].astype(dtype)
    s = sin[pos][:, None, :].astype(dtype)
    return partial_rope(y, c, s, rd)
