"""CPU pins of the attention oracle (no GPU).

The oracle is checked against (1) the reference's own unit tests, restated
with the reference's deterministic inputs (crates/inl-core/src/attention.rs
tests, crates/inl-text/src/gemma2.rs mask test, crates/inl-late/src/qwen3_5.rs
GQA-fold test), (2) closed forms that a wrong mask, sign or transpose breaks,
(3) a pure-Python brute force, and (4) packing invariance: for every form, the
packed variable-length oracle equals the reference's padded form on the real
rows.
"""
import math

import numpy as np
import pytest

from oracle import attention as oa

HEADS, KV_HEADS, DIM = 4, 2, 32  # attention.rs:319-321


def _t(shape, seed):
    return oa.pseudo(int(np.prod(shape)), seed).reshape(shape).astype(np.float32)


def _case(pads, seq):  # attention.rs:346-356
    b = len(pads)
    return (_t((b, HEADS, seq, DIM), 1), _t((b, KV_HEADS, seq, DIM), 2), _t((b, KV_HEADS, seq, DIM), 3))


def _max_diff_real(a, b, pads):
    return max(np.abs(a[r, :, p:] - b[r, :, p:]).max() for r, p in enumerate(pads))


def test_pseudo_matches_reference_lcg():
    # first values of the reference LCG, computed by hand from its constants
    state = (1 * 2654435761 + 1) & 0xFFFFFFFF
    state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
    assert oa.pseudo(1, 1)[0] == np.float32(state >> 8) / np.float32(1 << 24) - np.float32(0.5)
    v = oa.pseudo(10000, 3)
    assert v.min() >= -0.5 and v.max() < 0.5 and abs(v.mean()) < 0.02


def test_additive_mask_matches_the_reference_formula():
    """attention.rs:404-432 (seq 7, pads [0, 3, 7]): -1e4 per violated rule,
    summed."""
    seq, pads = 7, [0, 3, 7]
    mask = oa.qwen3_additive_mask(pads, seq)
    for row, pad in enumerate(pads):
        for q in range(seq):
            for k in range(seq):
                want = (-1e4 if k > q else 0.0) + (-1e4 if k < pad else 0.0)
                assert mask[row, 0, q, k] == want


def test_tiled_and_flash_match_eager_on_padded_batches():
    """attention.rs:435-445, in f32 arithmetic, bound 1e-5."""
    pads, seq = [0, 5, 11, 2], 13
    q, k, v = _case(pads, seq)
    mask = oa.qwen3_additive_mask(pads, seq, np.float32)
    scale = np.float32(DIM ** -0.5)
    eager = oa.qwen3_eager(q, k, v, mask, scale, HEADS // KV_HEADS).astype(np.float32)
    tiled = oa.qwen3_tiled(q, k, v, mask, scale, HEADS // KV_HEADS).astype(np.float32)
    flash = oa.qwen3_cpu_flash(q, k, v, pads, scale, dtype=np.float32)
    assert _max_diff_real(eager, tiled, pads) < 1e-5
    assert _max_diff_real(eager, flash, pads) < 1e-5


def test_tiling_is_exact_across_several_blocks():
    """attention.rs:448-481: 17 rows in tiles of 5."""
    pads, seq = [3, 0], 17
    q, k, v = _case(pads, seq)
    mask = oa.qwen3_additive_mask(pads, seq)
    ref = oa.qwen3_eager(q, k, v, mask, DIM ** -0.5, 2)
    blocks = oa.qwen3_tiled(q, k, v, mask, DIM ** -0.5, 2, tile=5)
    assert _max_diff_real(ref, blocks, pads) < 1e-5


def test_padding_does_not_change_real_rows():
    """attention.rs:484-531: a 9-token row alone and left-padded by 4."""
    q, k, v = _case([0], 9)
    z = lambda t: np.concatenate([np.zeros(t.shape[:2] + (4, DIM), np.float32), t], axis=2)
    alone = oa.qwen3_eager(q, k, v, oa.qwen3_additive_mask([0], 9), DIM ** -0.5, 2)
    inside = oa.qwen3_eager(z(q), z(k), z(v), oa.qwen3_additive_mask([4], 13), DIM ** -0.5, 2)[:, :, 4:]
    assert np.abs(alone - inside).max() < 1e-5


def test_packed_equals_left_padded_qwen3():
    """The drop-in claim for Qwen3: packed causal GQA == the reference's
    left-padded eager attention on every real row."""
    pads, seq = [0, 5, 11, 2], 13
    q, k, v = (t.astype(np.float64) for t in _case(pads, seq))
    ref = oa.qwen3_eager(q, k, v, oa.qwen3_additive_mask(pads, seq), DIM ** -0.5, 2)
    lens = [seq - p for p in pads]
    packed = oa.varlen_attention(oa.pack(q, lens, True), oa.pack(k, lens, True), oa.pack(v, lens, True),
                                 oa.cu_from_lengths(lens), causal=True, scale=DIM ** -0.5)
    assert np.abs(packed - oa.pack(ref, lens, True)).max() < 1e-12


def test_gemma2_mask_known_answers():
    """gemma2.rs:990-1003."""
    assert oa.gemma2_attention_mask([4, 4], 4, None) is None
    assert oa.gemma2_attention_mask([4], 4, 3) is None
    m = oa.gemma2_attention_mask([2, 4], 4, 1).reshape(2, 4, 4)
    ok = lambda r, q, k: m[r, q, k] == 0.0
    assert ok(0, 0, 1) and not ok(0, 0, 2) and not ok(0, 1, 3)
    assert ok(1, 2, 1) and ok(1, 2, 3) and not ok(1, 0, 2) and not ok(1, 3, 1)


@pytest.mark.parametrize("window", [None, 1, 3])
def test_packed_equals_right_padded_gemma2(window):
    """EmbeddingGemma 2: scale 1, -1e9 f32 mask, GQA 4/2, radius window."""
    lens, seq = [2, 6, 9], 9
    rng = np.random.default_rng(0)
    q = rng.standard_normal((3, 4, seq, 16)) * 0.3
    k = rng.standard_normal((3, 2, seq, 16)) * 0.3
    v = rng.standard_normal((3, 2, seq, 16))
    ref = oa.gemma2_attention(q, k, v, oa.gemma2_attention_mask(lens, seq, window))
    packed = oa.varlen_attention(oa.pack(q, lens, False), oa.pack(k, lens, False), oa.pack(v, lens, False),
                                 oa.cu_from_lengths(lens), causal=False,
                                 window=-1 if window is None else window, scale=1.0)
    assert np.abs(packed - oa.pack(ref, lens, False)).max() < 1e-12


@pytest.mark.parametrize("local", [False, True])
def test_packed_equals_right_padded_modernbert(local):
    """ModernBERT: q * 8^-1/2, -1e4 mask, local radius = local_attention/2."""
    lens, seq, half = [3, 17, 11], 17, 4
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((3, 4, seq, 8)) for _ in range(3))
    g, l = oa.modernbert_masks(lens, seq, half)
    ref = oa.modernbert_attend(q, k, v, l if local else g, 8 ** -0.5, tile=5)
    packed = oa.varlen_attention(*(oa.pack(t, lens, False) for t in (q, k, v)), oa.cu_from_lengths(lens),
                                 causal=False, window=half if local else -1, scale=8 ** -0.5)
    assert np.abs(packed - oa.pack(ref, lens, False)).max() < 1e-12


def test_qwen35_gqa_fold_matches_repeat_kv_across_tile_boundaries():
    """qwen3_5.rs:1014-1060: (b, kv, rep, t, d) = (2, 2, 3, 256 + 3, 8), pads
    of 0 and 1 key, causal and bidirectional, f32 bound 1e-5."""
    b, kv, rep, t, d = 2, 2, 3, oa.QUERY_TILE + 3, 8
    q = oa.pseudo(b * kv * rep * t * d, 20).reshape(b, kv * rep, t, d).astype(np.float64)
    k = oa.pseudo(b * kv * t * d, 21).reshape(b, kv, t, d).astype(np.float64)
    v = oa.pseudo(b * kv * t * d, 22).reshape(b, kv, t, d).astype(np.float64)
    for causal in (False, True):
        mask = np.zeros((b, 1, t, t))
        for bb in range(b):
            for row in range(t):
                for col in range(t):
                    if col >= t - bb - 1 or (causal and col > row):
                        mask[bb, 0, row, col] = -1e4
        scale = d ** -0.5
        scores = (q @ np.swapaxes(oa.repeat_kv(k, rep), 2, 3)) * scale + mask
        expected = oa.softmax_last(scores) @ oa.repeat_kv(v, rep)
        actual = oa.qwen35_grouped_tiled(q, k, v, mask, scale, rep)
        assert np.abs(actual - expected).max() < 1e-5
    # and the packed form equals it on real rows (keys past each length masked)
    lens = [t - 1, t - 2]
    m = oa.qwen35_mask(lens, t, True)
    ref = oa.qwen35_grouped_tiled(q, k, v, m, d ** -0.5, rep)
    packed = oa.varlen_attention(*(oa.pack(x[:, :, :], lens, False) for x in (q, k, v)),
                                 oa.cu_from_lengths(lens), causal=True, scale=d ** -0.5)
    assert np.abs(packed - oa.pack(ref, lens, False)).max() < 1e-12


def test_packed_equals_vision_key_padding():
    """vision.rs:226-259: scale 1, -1e9 on padding keys only."""
    lens, seq = [5, 12], 12
    rng = np.random.default_rng(2)
    q, k, v = (rng.standard_normal((2, 3, seq, 8)) * 0.5 for _ in range(3))
    pad = np.array([[0] * l + [1] * (seq - l) for l in lens])
    ref = oa.vision_masked_attention(q, k, v, oa.vision_key_mask(pad), tile=5)
    packed = oa.varlen_attention(*(oa.pack(t, lens, False) for t in (q, k, v)), oa.cu_from_lengths(lens),
                                 causal=False, scale=1.0)
    assert np.abs(packed - oa.pack(ref, lens, False)).max() < 1e-12


@pytest.mark.parametrize("causal,window", [(True, -1), (False, -1), (False, 2), (True, 3)])
def test_zero_queries_give_means_of_visible_values(causal, window):
    """q = 0 makes every visible key equally likely, so each output row is the
    plain mean of the V rows its mask admits: causal prefixes, window bands."""
    lens = [1, 4, 9]
    n = sum(lens)
    rng = np.random.default_rng(3)
    k, v = rng.standard_normal((n, 1, 4)), rng.standard_normal((n, 1, 4))
    out = oa.varlen_attention(np.zeros((n, 2, 4)), k, v, oa.cu_from_lengths(lens), causal=causal,
                              window=window, scale=1.0)
    start = 0
    for t in lens:
        for i in range(t):
            lo = 0 if window < 0 else max(0, i - window)
            hi = i + 1 if causal else t
            if window >= 0:
                hi = min(hi, i + window + 1)
            want = v[start + lo:start + hi, 0].mean(axis=0)
            assert np.allclose(out[start + i, 0], want) and np.allclose(out[start + i, 1], want)
        start += t


def test_brute_force_python_softmax():
    """Scalar Python loops (math.exp), GQA head mapping h -> h // 2, causal."""
    rng = np.random.default_rng(4)
    lens, hq, hkv, d = [3, 5], 4, 2, 3
    n = sum(lens)
    q, k, v = rng.standard_normal((n, hq, d)), rng.standard_normal((n, hkv, d)), rng.standard_normal((n, hkv, d))
    out = oa.varlen_attention(q, k, v, oa.cu_from_lengths(lens), causal=True, scale=0.7)
    start = 0
    for t in lens:
        for i in range(t):
            for h in range(hq):
                kh = h // (hq // hkv)
                s = [0.7 * sum(q[start + i, h, e] * k[start + j, kh, e] for e in range(d)) for j in range(i + 1)]
                mx = max(s)
                w = [math.exp(x - mx) for x in s]
                z = sum(w)
                for e in range(d):
                    want = sum(w[j] * v[start + j, kh, e] for j in range(i + 1)) / z
                    assert abs(out[start + i, h, e] - want) < 1e-12
        start += t


def test_single_token_text_returns_its_value():
    v = np.random.default_rng(5).standard_normal((1, 2, 8))
    out = oa.varlen_attention(np.ones((1, 4, 8)), np.ones((1, 2, 8)), v, [0, 1], causal=True, scale=1.0)
    assert np.allclose(out[0, :2], v[0, 0]) and np.allclose(out[0, 2:], v[0, 1])


def test_visible_pair_counts():
    rng = np.random.default_rng(6)
    for t in [1, 2, 7, 64, 300]:
        assert oa.visible_pairs([t], True) == t * (t + 1) // 2
        assert oa.visible_pairs([t], False) == t * t
        for w in [0, 1, 5, 64]:
            assert oa.visible_pairs([t], False, w) == int(oa.allowed(t, t, False, w).sum())
            assert oa.visible_pairs([t], True, w) == int(oa.allowed(t, t, True, w).sum())
    assert oa.attention_flops([3, 4], 2, 8, True) == 4 * 2 * 8 * (6 + 10)


def test_workload_generators_reproduce_the_measurement_plan():
    from inl_hip import workloads as w
    lens = w.qwen3_op_lengths()
    assert (len(lens), sum(lens)) == (713, 200179)
    assert len(w.batches(lens)) == 12
    assert abs(oa.attention_flops(lens, 16, 128, True) / 1e12 - 0.50343) < 1e-4
    assert sum(w.uniform_lengths(32, 64, 8192)) == 139124
    assert sum(w.uniform_lengths(128, 32, 2048)) == 135892
    assert sum(w.uniform_lengths(8, 16, 256)) == 778


def test_c_restatement_agrees_with_numpy_oracle():
    """oracle/attn_ref.c (f32, online softmax over 64-key blocks) is an
    independent second implementation."""
    from oracle import cref
    rng = np.random.default_rng(7)
    lens = [1, 5, 64, 100, 257]
    n = sum(lens)
    q = rng.standard_normal((n, 8, 64)).astype(np.float32)
    k = rng.standard_normal((n, 2, 64)).astype(np.float32)
    v = rng.standard_normal((n, 2, 64)).astype(np.float32)
    cu = oa.cu_from_lengths(lens)
    for causal, win in [(True, -1), (False, -1), (False, 20), (True, 7)]:
        a = cref.attention_f32(q, k, v, cu, causal=causal, window=win, scale=0.125)
        b = oa.varlen_attention(q, k, v, cu, causal=causal, window=win, scale=0.125)
        assert np.abs(a - b).max() < 1e-5
