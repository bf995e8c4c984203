"""CPU pins of the prologue and pooling oracles (no GPU): the reference's
own unit tests (RoPE fused == manual half-split, RMSNorm == textbook, SPLADE
known answers and formula tests, SparseVector::from_pairs, Matryoshka), plus
invariants a wrong index or sign breaks (RoPE is a norm-preserving rotation
whose scores depend only on relative position)."""
import numpy as np
import pytest

from oracle import attention as oa
from oracle import pooling as opl
from oracle import prologue as op


def _pseudo7(n, seed):  # the qwen3/mod.rs test variant of the LCG
    return oa.pseudo(n, seed, offset=7)


def test_fused_rope_matches_manual_half_split_qwen3():
    """qwen3/mod.rs:678-703: heads 2, seq 5, dim 32, theta 1e4, pseudo seed 11."""
    heads, seq, dim = 2, 5, 32
    x = _pseudo7(heads * seq * dim, 11).reshape(1, heads, seq, dim).astype(np.float64)
    c, s = op.rope_table(dim, 10_000.0, seq)
    fused = op.rope(x, c.astype(np.float64), s.astype(np.float64))
    manual = op.rope_manual(x, c.astype(np.float64), s.astype(np.float64))
    assert np.abs(fused - manual).max() < 1e-12


def test_fused_rope_matches_manual_half_split_gemma2():
    """gemma2.rs:916-939: x = (i % 17) * 0.05 - 0.4, head_dim 16, seq 5."""
    hd, seq = 16, 5
    x = np.array([(i % 17) * 0.05 - 0.4 for i in range(2 * seq * hd)]).reshape(1, 2, seq, hd)
    c, s = op.rope_table(hd, 10_000.0, seq)
    assert np.abs(op.rope(x, c, s) - op.rope_manual(x, c, s)).max() < 1e-6


def test_rope_is_a_rotation_and_depends_on_relative_position():
    """Norm preserved per pair; position 0 is the identity; q.k after RoPE at
    positions (i, j) depends only on i - j - the property that makes a packed
    text (positions from 0) equal to the reference's left-padded one."""
    rng = np.random.default_rng(0)
    d = 64
    c, s = op.rope_table(d, 1e6, 40)
    c, s = c.astype(np.float64), s.astype(np.float64)
    x = rng.standard_normal((40, d))
    y = op.rope(x, c, s)
    h = d // 2
    assert np.allclose(x[:, :h] ** 2 + x[:, h:] ** 2, y[:, :h] ** 2 + y[:, h:] ** 2)
    assert np.allclose(y[0], x[0])
    q, k = rng.standard_normal(d), rng.standard_normal(d)
    rot = lambda v, p: op.rope(v[None], c[p:p + 1], s[p:p + 1])[0]
    dots = [rot(q, i + 7) @ rot(k, i) for i in range(20)]
    assert np.allclose(dots, dots[0], atol=1e-9)


def test_rms_norm_textbook_and_unit_rms():
    """qwen3/mod.rs:706-730 inputs (pseudo seeds 9 and 4); with unit weight the
    output has mean square mean(x^2) / (mean(x^2) + eps)."""
    x = _pseudo7(3 * 48, 9).reshape(3, 48).astype(np.float64)
    w = _pseudo7(48, 4).astype(np.float64)
    y = op.rms_norm(x, w, 1e-6)
    ms = (x * x).mean(-1, keepdims=True)
    assert np.abs(y - x / np.sqrt(ms + 1e-6) * w).max() < 1e-12
    u = op.rms_norm(x, None, 1e-6)
    assert np.allclose((u * u).mean(-1), ms[:, 0] / (ms[:, 0] + 1e-6))


def test_library_rope_tables_match_reference_construction():
    """inl_rope_table_host mode 0 (f64 angles) is bit-identical to the oracle;
    mode 1 (f32, Qwen3.5) agrees to a few f32 ulps (libm vs numpy cos)."""
    import inl_hip
    for dim, theta, n in [(128, 1e6, 300), (256, 1e4, 64), (64, 160000.0, 100)]:
        c, s = inl_hip.rope_table(dim, theta, n, 0)
        rc, rs = op.rope_table(dim, theta, n)
        assert np.array_equal(c, rc) and np.array_equal(s, rs)
    c, s = inl_hip.rope_table(64, 1e7, 200, 1)
    rc, rs = op.rope_table_f32(64, 1e7, 200)
    assert np.abs(c - rc).max() < 1e-5 and np.abs(s - rs).max() < 1e-5


def test_positions_restart_per_text():
    import inl_hip
    assert inl_hip.positions([0, 3, 3, 5]).tolist() == [0, 1, 2, 0, 1]
    assert op.positions_of([0, 3, 3, 5]).tolist() == [0, 1, 2, 0, 1]


# ---- SPLADE (crates/inl-sparse/src/modernbert.rs tests) ----

def _pool(logits, rows, prefix, masked, canon, shift):
    idx, ends = opl.speakers(rows, prefix, seq=logits.shape[1])
    return opl.splade_pool(logits.reshape(-1, logits.shape[2])[idx], ends, None, shift, masked, canon)


def test_splade_shift_relu_log1p_max():
    """modernbert.rs:1299-1309."""
    out = _pool(np.array([[[3.0, 0.5, 1.5], [0.0, 0.9, 4.0]]], np.float32), [[5, 6]], [], [], None, 1.0)
    assert abs(out[0, 0] - np.log(3)) < 1e-6 and out[0, 1] == 0 and abs(out[0, 2] - np.log(4)) < 1e-6


def test_splade_prefix_and_masked_terms():
    """modernbert.rs:1311-1322."""
    out = _pool(np.array([[[50.0, 50.0, 50.0], [1.0, 0.0, 30.0]]], np.float32), [[9, 5]], [9], [2], None, 0.0)
    assert abs(out[0, 0] - np.log(2)) < 1e-6 and out[0, 1] == 0 and out[0, 2] == 0


def test_splade_positions_beyond_length_ignored():
    """modernbert.rs:1324-1334."""
    out = _pool(np.array([[[1.0, 0.0], [99.0, 99.0]]], np.float32), [[5]], [], [], None, 0.0)
    assert abs(out[0, 0] - np.log(2)) < 1e-6 and out[0, 1] == 0


def test_splade_canonical_fold():
    """modernbert.rs:1336-1345."""
    out = _pool(np.array([[[1.0, 5.0, 3.0]]], np.float32), [[5]], [], [], [0, 1, 0], 0.0)
    assert out.shape == (1, 2)
    assert abs(out[0, 0] - np.log(4)) < 1e-6 and abs(out[0, 1] - np.log(6)) < 1e-6


def test_splade_random_logits_match_plain_formula():
    """modernbert.rs:1347-1393: xorshift logits in [-3, 5), ragged rows, prefix
    id 9, masked terms {3, 11}, shift 1.5, checked term by term against
    max over real non-prefix positions of ln(1 + relu(logit - shift))."""
    batch, seq, vocab = 3, 9, 17
    state = 0x2545F4914F6CDD1D
    vals = []
    for _ in range(batch * seq * vocab):
        state ^= (state << 13) & 0xFFFFFFFFFFFFFFFF
        state ^= state >> 7
        state ^= (state << 17) & 0xFFFFFFFFFFFFFFFF
        vals.append(np.float32((state >> 40) / float(1 << 24)) * np.float32(8.0) - np.float32(3.0))
    logits = np.array(vals, np.float32).reshape(batch, seq, vocab)
    rows = [[9, 5, 6, 7, 8, 5, 6, 7, 8], [9, 5, 6], [5]]
    got = _pool(logits, rows, [9], [3, 11], None, 1.5)
    for r, ids in enumerate(rows):
        for t in range(vocab):
            want = 0.0
            if t not in (3, 11):
                for p, tok in enumerate(ids):
                    if tok != 9:
                        want = max(want, float(np.log(max(logits[r, p, t] - 1.5, 0.0) + 1.0)))
            assert abs(got[r, t] - want) < 1e-5


def test_sparse_from_pairs_drops_unusable_weights():
    """lib.rs:286-297 semantics on a dense row: keep finite, positive."""
    idx, val = opl.sparse_from_pairs([0.0, 0.0, 0.0, 0.5, 0.0, 0.0, -1.0, 2.5, np.nan])
    assert idx.tolist() == [3, 7] and val.tolist() == [0.5, 2.5]


def test_matryoshka_truncate_and_normalize():
    v = np.array([3.0, 4.0, 12.0], np.float32)
    out = opl.truncate_and_normalize(v, 2)
    assert np.allclose(out, [0.6, 0.8])
    assert np.array_equal(opl.truncate_and_normalize(np.zeros(4, np.float32), 2), np.zeros(2, np.float32))


def test_last_and_mean_pool_closed_forms():
    h = np.arange(12, dtype=np.float64).reshape(6, 2)
    cu = [0, 2, 2, 6]
    m = opl.mean_pool(h, cu)
    assert np.allclose(m, [[1, 2], [0, 0], [7, 8]])
    last = opl.last_token(h, [0, 2, 6], None, 0.0)
    for row, src in zip(last, [h[1], h[5]]):
        assert np.allclose(row, src / np.linalg.norm(src))
